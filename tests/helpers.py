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

    |actual - expected| <= 2^-8 * |expected| + 2.5e-4 * max|expected| + 1e-6:
    half an output ulp (bf16: <= 2^-8 relative; fp16 outputs are held to the same
    term) plus the accumulation error relative to the row scale: the FP8 MFMA
    truncates its partial sums (~2^-13 below the largest product), so the fp32
    accumulators and the row mass are not exact sums (the deferred mean restore's
    weights enter as fp16 hi + lo parts, about 22 bits). Measured beyond the half ulp,
    as a fraction of the row's largest output: at most 6.4e-5 on [1,2,4096..37741,
    64/128] inputs (N(0,1), outlier K / clustered V with smoothing, Student-t, both
    probability paths, bf16 and fp16) and 1.0e-4 on [1,2,75482,128] with smoothing;
    the bound allows 2.5e-4.
    """
    e = np.asarray(expected, np.float64)
    a = np.asarray(actual, np.float64)
    scale = np.abs(e).max(axis=-1, keepdims=True)
    bound = 2.0 ** -8 * np.abs(e) + 2.5e-4 * scale + 1e-6
    return np.abs(a - e), bound


# Scales and dot products for which the last tile's rounding order
# RN(RN(float(acc)*RN(qs*ks))*sm) and the other tiles' RN(float(acc)*RN(sm*RN(qs*ks)))
# give different ExpCast bytes for key 1 (sm = RN(128^-0.5)); found by search.
ORDER_QS = float.fromhex("0x1.b2c8f2p-2")
ORDER_KS = float.fromhex("0x1.3a883p-1")
ORDER_ACC = (15989, 15902)
ORDER_CODE_LAST, ORDER_CODE_OTHER = 96, 97


def rounding_order_payload(nk):
    """Payload state (D=128, one query row of ones) whose keys 0 and 1 have dot products
    ORDER_ACC; every other key is zero. With nk <= 128 the pair sits in the last tile,
    with nk > 128 in a tile before the last."""
    dim, tiles = 128, (nk + 127) // 128
    q = np.ones((1, 1, 1, dim), np.int8)
    k = np.zeros((1, 1, nk, dim), np.int8)
    for key, acc in enumerate(ORDER_ACC):
        k[0, 0, key, :125] = 127
        k[0, 0, key, 125] = acc - 125 * 127
    qs = np.ones((1, 1, 32), np.float32)
    qs[0, 0, 0] = ORDER_QS
    ks = np.ones((1, 1, tiles * 4), np.float32)
    ks[0, 0, 0] = ORDER_KS
    return {"q": q, "k": k, "v": np.zeros((1, 1, dim, tiles * 128), np.uint8), "qs": qs, "ks": ks,
            "vs": np.ones((1, 1, dim), np.float32), "means": None, "expcast": True, "block_values": False,
            "scale": float(np.float32(dim ** -0.5)), "output_type": 1}


# A one-row payload (D=64, two tiles) where the folded ExpCast encode of the reference's
# default kernel modes (sal/csrc/vc/vc_math.cuh:76-111) and the unfused encode give
# different bytes for key 96 of the first tile (found by search): key 45 holds the row
# maximum (byte 120); key 96 is 116 unfused and 115 folded.
FOLD_Q = (-115, -105, 3, -123)
FOLD_K = {45: (25, -117, 79, -112), 96: (-56, 8, -96, -119)}
FOLD_QS = float.fromhex("0x1.6f324p-7")
FOLD_KS = tuple(float.fromhex(x) for x in ("0x1.55ded6p-7", "0x1.90b75ap-7", "0x1.4523e2p-6", "0x1.12c5fep-6",
                                              "0x1.0756f6p-6", "0x1.2fd4d6p-6", "0x1.078d94p-6", "0x1.6e4c06p-8"))
FOLD_CODE_UNFUSED, FOLD_CODE_FOLDED = 116, 115


def folded_encode_payload(extreme_rows=(), nq=32):
    """FOLD_* on query row 0 of an nq-row payload; every row in `extreme_rows` gets a
    row maximum far above 128 (the folded encode's safety bound), which makes its whole
    16-row group fall back to the unfused encode."""
    dim, nk = 64, 200
    q = np.zeros((1, 1, nq, dim), np.int8)
    k = np.zeros((1, 1, nk, dim), np.int8)
    q[0, 0, 0, :4] = FOLD_Q
    for key, row in FOLD_K.items():
        k[0, 0, key, :4] = row
    qs = np.ones((1, 1, ((nq + 63) // 64) * 32), np.float32)
    qs[0, 0, 0] = FOLD_QS
    for r in extreme_rows:
        q[0, 0, r, 0] = 127
        qs[0, 0, (r // 16) * 8 + r % 8] = 100.0
    ks = np.asarray(FOLD_KS, np.float32).reshape(1, 1, 8)
    return {"q": q, "k": k, "v": np.zeros((1, 1, dim, 256), np.uint8), "qs": qs, "ks": ks,
            "vs": np.ones((1, 1, dim), np.float32), "means": None, "expcast": True, "block_values": False,
            "scale": float(np.float32(dim ** -0.5)), "output_type": 1}
