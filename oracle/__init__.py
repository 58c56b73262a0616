"""CPU oracle for the attention hot path and its RoPE producer — TEST INFRASTRUCTURE, never a product path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import, call, link or execute anything in this package, and only to check results against
(or as the timed CPU baseline) — the ``fast_infer_amd`` package never does.

Contents (each function cites the reference file:line it restates):

* ``attention`` — fp32 closed forms of causal GQA prefill and paged decode, and
  numpy restatements of the reference's Triton tile loops (same tile sizes, same
  online-softmax update order) for bit-level comparison with the reference's own
  outputs.
* ``kv`` — pure-Python restatement of the KV pool writes (model.py:162-201,
  kv_cache.py:69-103) and of the block allocator (kv_cache.py:12-113).
* ``rope`` — numpy restatement of the RoPE table and of its fp16 application
  (kernels/rope.py:9-44), and of RoPE followed by the pool write (model.py:101,
  :117, :120).
* ``block_manager`` — the reference allocator driven with per-row token counts, plus
  row release (the device block manager's checker).
* ``int4`` — numpy restatement of the INT4 weight format: quantize (loader.py:9-41),
  unpack / dequantize (matmul.py:309-326), and the float64 product with its error bound.
* ``rmsnorm`` — RMSNorm (kernels/rms_norm.py:8-43) in float64 and its fp16 error bound.
* ``ref_algo.c`` (+ ``native``) — the same tile algorithms in C with OpenMP, used
  as the CPU baseline ("port").

How each function is pinned (golden vectors from the reference kernels, closed
forms, invariants, brute force) is listed in each module's docstring.
"""
