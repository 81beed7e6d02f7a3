"""Shared helpers for the parity tests: seeded inputs, layout conversions, metrics."""
import numpy as np
import torch


def make_qkv(B, H, Nq, Nk, D, dtype=torch.bfloat16, seed=0, kind="normal"):
    """Seeded CPU inputs (q, then k, then v), cast to the input dtype.

    kind="normal": i.i.d. N(0,1).
    kind="outlier": Q N(0,1); K = N(0,1) + per-(head, channel) offset with variance 4;
      V = one of 8 per-head centroids (variance 2) + N(0, variance 0.3) noise.
    kind="student": Q, K = 0.5 * Student-t(nu=4) (numpy PCG64), V N(0,1).
    """
    g = torch.Generator().manual_seed(seed)
    if kind == "normal":
        q = torch.randn(B, H, Nq, D, generator=g)
        k = torch.randn(B, H, Nk, D, generator=g)
        v = torch.randn(B, H, Nk, D, generator=g)
    elif kind == "outlier":
        q = torch.randn(B, H, Nq, D, generator=g)
        k = torch.randn(B, H, Nk, D, generator=g) + torch.randn(B, H, 1, D, generator=g) * 2.0
        cent = torch.randn(B, H, 8, D, generator=g) * 2.0 ** 0.5
        assign = torch.randint(0, 8, (B, H, Nk), generator=g)
        v = torch.gather(cent, 2, assign[..., None].expand(B, H, Nk, D)) + torch.randn(B, H, Nk, D, generator=g) * 0.3 ** 0.5
    elif kind == "student":
        rng = np.random.Generator(np.random.PCG64(seed))
        q = torch.from_numpy(0.5 * rng.standard_t(4, size=(B, H, Nq, D))).float()
        k = torch.from_numpy(0.5 * rng.standard_t(4, size=(B, H, Nk, D))).float()
        v = torch.randn(B, H, Nk, D, generator=g)
    else:
        raise ValueError(kind)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def bits(x):
    """16-bit tensor -> numpy uint16 bit patterns (contiguous)."""
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def dtype_name(dtype):
    return {torch.bfloat16: "bfloat16", torch.float16: "float16"}[dtype]


def storage_to_logical(v8, value_token):
    """[B,H,D,tiles*128] payload in storage order -> logical token order (numpy uint8)."""
    arr = v8.view(torch.uint8).cpu().numpy() if torch.is_tensor(v8) else v8
    B, H, D, npad = arr.shape
    tiles = npad // 128
    tok = np.asarray(value_token)
    inv = np.empty(128, np.int64)
    inv[tok] = np.arange(128)
    return arr.reshape(B, H, D, tiles, 128)[..., inv].reshape(B, H, D, npad)


def logical_to_storage(v8, value_token):
    B, H, D, npad = v8.shape
    tok = np.asarray(value_token)
    return np.ascontiguousarray(v8.reshape(B, H, D, npad // 128, 128)[..., tok].reshape(B, H, D, npad))


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-300))


def output_bound(actual, expected):
    """Elementwise tolerance of the bf16/fp16 output vs the fp32-simulated oracle.

    |actual - expected| <= 2^-7 * |expected| + 2e-3 * max|expected| + 1e-6:
    one output ulp (bf16 ulp <= 2^-7 relative) plus the FP8 MFMA accumulation
    error (chunks truncated ~2^-13 below their largest product) relative to the
    row scale.
    """
    e = np.asarray(expected, np.float64)
    a = np.asarray(actual, np.float64)
    scale = np.abs(e).max(axis=-1, keepdims=True)
    bound = 2.0 ** -7 * np.abs(e) + 2e-3 * scale + 1e-6
    return np.abs(a - e), bound
