"""MI355X roofline constants and the algorithmic work of the attention path.

Peaks are MI355X's published dense figures for one GPU.  The work formulas count
what the algorithm must move or compute, independent of how a kernel does it:

* paged decode — every context token's K and V row of every kv head once (4 KiB per
  token at 8 kv heads x 128 dims x fp16 x 2), plus q and o, plus the block-table
  entries covering the context;
* causal prefill — 4 * B * H * S^2 * D / 2 flops (QK^T and PV over the causal half);
* INT4 linear layer — packed weights (K/2 bytes per row) and fp16 scales (2 bytes per
  128-group) read once, X read once, the fp16 output written once; 2 * M * N * K flops;
* fused RoPE + KV write — q, k, v rows read once, the cos/sin rows of the distinct
  positions read once, rotated q (and k when returned) written once, k and v rows
  written into the pool once.
"""

from __future__ import annotations

import math

HBM_PEAK_GBS = 8000.0            # HBM3E, GB/s
FP16_MFMA_PEAK_TFLOPS = 2516.6   # dense fp16 MFMA, TFLOP/s (256 CU x 2.4 GHz x 4096 flop/clk)


def decode_bytes(context_lens, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 block_size: int) -> int:
    """Algorithmic HBM bytes of one decode call over rows with these context lengths."""
    lens = [int(c) for c in context_lens]
    kv = sum(lens) * num_kv_heads * head_dim * 2 * 2
    qo = 2 * len(lens) * num_q_heads * head_dim * 2
    table = 4 * sum(math.ceil(c / block_size) for c in lens)
    return kv + qo + table


def prefill_flops(batch: int, num_heads: int, seq_len: int, head_dim: int) -> float:
    """Algorithmic flops of causal attention (QK^T + PV over the causal half)."""
    return 4.0 * batch * num_heads * seq_len * seq_len * head_dim / 2.0


def prefill_scatter_bytes(batch: int, seq_len: int, num_kv_heads: int, head_dim: int) -> int:
    """Bytes the fused K/V pool write stores (K and V rows of every token)."""
    return batch * seq_len * num_kv_heads * head_dim * 2 * 2


def rope_store_bytes(batch: int, tokens: int, num_q_heads: int, num_kv_heads: int,
                     head_dim: int, positions: int, pool: bool, return_k: bool) -> int:
    """Algorithmic HBM bytes of one fused RoPE (+ pool write) call; ``positions`` is the
    number of distinct table rows the call touches."""
    row = head_dim * 2
    n = batch * tokens
    read = n * (num_q_heads + num_kv_heads + (num_kv_heads if pool else 0)) * row
    read += positions * row * 2
    write = n * num_q_heads * row
    write += n * num_kv_heads * row * ((1 if return_k else 0) + (2 if pool else 0))
    return read + write


def int4_matmul_bytes(M: int, N: int, K: int, groupsize: int = 128) -> int:
    """Algorithmic HBM bytes of one INT4 linear-layer call."""
    return N * K // 2 + N * (K // groupsize) * 2 + M * K * 2 + M * N * 2


def matmul_flops(M: int, N: int, K: int) -> float:
    return 2.0 * M * N * K
