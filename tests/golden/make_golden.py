"""Write golden vectors from the reference's own attention kernels.

Runs Fast_Infer's ``flash_attention`` and ``paged_attention``
(kernels/attention.py:80-113, :191-233) from the read-only reference checkout under
``TRITON_INTERPRET=1`` on CPU tensors, for the seeded inputs of ``specs.py``, and
stores their fp16 outputs in ``attention_golden.npz`` plus the input hashes and
provenance in ``attention_golden.json``.  Prefill is called the way the reference
model calls it: q/k/v as [B, H, S, D] views of [B, S, H, D] tensors, with K/V
expanded by ``repeat_interleave`` (model.py:104-113).  Ragged decode is one call per
row (batch 1, num_tokens = ctx_b), since the reference has no per-row lengths.

Only the attention kernels are run: the KV writes and the allocator are pinned by
brute force in the tests and are not executed from the reference.

Usage (this container only; the reference does not exist on the GPU box):
    python tests/golden/make_golden.py [/root/reference]
"""

from __future__ import annotations

import importlib.util
import json
import os
import sys
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"
sys.dont_write_bytecode = True

import numpy as np  # noqa: E402
import torch  # noqa: E402

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import specs  # noqa: E402


def load_reference(root: Path):
    spec = importlib.util.spec_from_file_location(
        "fast_infer_reference_attention", root / "kernels" / "attention.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main(root: str = "/root/reference") -> None:
    import triton

    ref = load_reference(Path(root))
    arrays: dict[str, np.ndarray] = {}
    meta = {"generator": "tests/golden/make_golden.py",
            "reference": "kernels/attention.py (flash_attention, paged_attention)",
            "mode": "TRITON_INTERPRET=1 on CPU", "triton": triton.__version__,
            "torch": torch.__version__, "cases": {}}

    for name, sp in specs.DECODE_CASES.items():
        q, kc, vc, table, lens = specs.decode_inputs(sp)
        out = ref.paged_attention(q, kc, vc, table, sp["bs"], sp["ctx"])
        arrays[f"{name}__out"] = out.numpy()
        meta["cases"][name] = {"kind": "decode", "spec": sp,
                               "inputs_sha256": specs.sha256(q, kc, vc, table)}
        print(name, tuple(out.shape))

    for name, sp in specs.RAGGED_CASES.items():
        q, kc, vc, table, lens = specs.decode_inputs(sp)
        rows = []
        for b, n in enumerate(lens):
            rows.append(ref.paged_attention(q[b:b + 1], kc, vc, table[b:b + 1], sp["bs"], n))
        out = torch.cat(rows, 0)
        arrays[f"{name}__out"] = out.numpy()
        meta["cases"][name] = {"kind": "ragged", "spec": sp,
                               "inputs_sha256": specs.sha256(q, kc, vc, table)}
        print(name, tuple(out.shape))

    for name, sp in specs.PREFILL_CASES.items():
        q, k, v = specs.prefill_inputs(sp)
        G = sp["H"] // sp["Hkv"]
        out = ref.flash_attention(q, k.repeat_interleave(G, dim=1), v.repeat_interleave(G, dim=1))
        rows = specs.prefill_rows(sp)
        arrays[f"{name}__out"] = out[:, :, rows].numpy()
        arrays[f"{name}__rows"] = rows.astype(np.int32)
        meta["cases"][name] = {"kind": "prefill", "spec": sp,
                               "inputs_sha256": specs.sha256(q, k, v)}
        print(name, tuple(out.shape), "kept rows", len(rows))

    np.savez_compressed(HERE / "attention_golden.npz", **arrays)
    (HERE / "attention_golden.json").write_text(json.dumps(meta, indent=1, sort_keys=True))


if __name__ == "__main__":
    main(*sys.argv[1:])
