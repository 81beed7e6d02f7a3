"""Write golden vectors for the Sage per-thread INT8 quantizer.

No test in the reference pins the INT8 bytes of ``per_thread_int8``
(third_party/sageattention_local/sageattention_local/triton/quant_per_thread.py:154-204),
so this script runs that function from the reference checkout under Triton's
interpreter (TRITON_INTERPRET=1: numpy semantics, IEEE division) on small
seeded inputs and stores inputs and outputs as a fixture. It pins the
quantizer's formula (scale, +-0.5, truncation, row/key grouping, padding),
not the H200 GPU lowering of its division.

Run in the build container only (needs /root/reference):
    python tests/golden/make_int8_vectors.py
Output: tests/golden/int8_per_thread.npz
"""
import importlib.util
import os
import sys
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402
import torch  # noqa: E402

REF = Path("/root/reference/third_party/sageattention_local/sageattention_local/triton/quant_per_thread.py")
OUT = Path(__file__).resolve().parent / "int8_per_thread.npz"

CASES = [  # (B, H, Nq, Nk, D, dtype, seed)
    (1, 2, 130, 257, 128, torch.bfloat16, 11),
    (1, 1, 64, 128, 64, torch.bfloat16, 12),
    (2, 1, 17, 5, 128, torch.float16, 13),
    (1, 1, 200, 300, 64, torch.float16, 14),
]


def main():
    spec = importlib.util.spec_from_file_location("ref_quant_per_thread", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    arrays = {}
    for i, (B, H, Nq, Nk, D, dtype, seed) in enumerate(CASES):
        g = torch.Generator().manual_seed(seed)
        q = (torch.randn(B, H, Nq, D, generator=g) * 2).to(dtype)
        k = (torch.randn(B, H, Nk, D, generator=g) + torch.randn(B, H, 1, D, generator=g)).to(dtype)
        # Exact multiples of a power of two make x/s land on .5 boundaries often.
        q[..., 0, :8] = torch.tensor([127, -127, 63.5, -63.5, 0.5, -0.5, 1.5, 0], dtype=dtype)
        km = k.mean(dim=2, keepdim=True)
        q8, qs, k8, ks = mod.per_thread_int8(q, k, km, BLKQ=64, WARPQ=16, BLKK=128, WARPK=128,
                                             tensor_layout="HND")
        view = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
        arrays[f"c{i}_q"] = view(q)
        arrays[f"c{i}_k"] = view(k)
        arrays[f"c{i}_km"] = view(km)
        arrays[f"c{i}_q8"] = q8.numpy()
        arrays[f"c{i}_qs"] = qs.numpy()
        arrays[f"c{i}_k8"] = k8.numpy()
        arrays[f"c{i}_ks"] = ks.numpy()
        arrays[f"c{i}_meta"] = np.array([B, H, Nq, Nk, D, 1 if dtype == torch.bfloat16 else 0, seed], np.int64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({len(CASES)} cases)")


if __name__ == "__main__":
    sys.exit(main())
