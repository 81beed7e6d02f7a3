"""CPU oracle for the sageattn_vc contract (numpy + the C restatement in vc_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package. The functions keep
the reference's names and argument meaning so the parity tests read like the
reference's own tests:

* ``expcast_codes``      -- sal/sageattention_local/vc_reference.py:9-11
* ``value_permutation``  -- sal/sageattention_local/vc_reference.py:14-17 (Sage layout)
* ``group_values``       -- sal/csrc/vc/clustering.cu:140-167, pybind.cpp:39-44
* ``per_thread_int8``    -- sal/sageattention_local/triton/quant_per_thread.py:154-204
* ``per_channel_fp8``    -- sal/sageattention_local/quant.py:224-293
* ``prepare_values``     -- sal/csrc/vc/preprocess.cu:138-168
* ``prepare``            -- sal/sageattention_local/vc.py:141-170
* ``reference``          -- sal/sageattention_local/vc_reference.py:20-91

("sal/" abbreviates third_party/sageattention_local/ of the reference.)
Arrays are numpy; 16-bit inputs are passed as raw uint16 bit patterns plus a
dtype tag ("bfloat16" or "float16"). V payloads are LOGICAL: [B,H,D,tiles*128]
in token order (the reference stores the Sage 16-token permutation instead;
``value_permutation`` converts).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "lib" / "libvc_oracle.so"
_lib = None

DTYPES = {"float16": 0, "bfloat16": 1}


def build(force: bool = True) -> Path:
    """Compile vc_oracle.c with gcc (no FMA contraction, IEEE semantics)."""
    if _LIB_PATH.exists() and not force:
        return _LIB_PATH
    _LIB_PATH.parent.mkdir(parents=True, exist_ok=True)
    tmp = _LIB_PATH.with_suffix(".so.tmp%d" % os.getpid())
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-fopenmp", "-Wall", "-o", str(tmp), str(_HERE / "vc_oracle.c"), "-lquadmath", "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, _LIB_PATH)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(L):
    P = ctypes.c_void_p
    i64, i32, f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_float
    L.vco_expcast_code.restype = ctypes.c_uint8
    L.vco_expcast_code.argtypes = [f32]
    L.vco_exp2_rn.restype = f32
    L.vco_exp2_rn.argtypes = [f32]
    L.vco_fp8_exp2_sweep.argtypes = [ctypes.c_uint32, i64, P]
    L.vco_fp8_exp2_sweep.restype = None
    for name in ("vco_expcast_codes", "vco_e4m3_encode_array", "vco_e4m3_decode_array",
                 "vco_cvt_u8_array", "vco_fp8_exp2_codes"):
        getattr(L, name).argtypes = [P, P, i64]
        getattr(L, name).restype = None
    L.vco_tile_tree_sum.restype = ctypes.c_double
    L.vco_tile_tree_sum.argtypes = [P]
    L.vco_linspace_ids.argtypes = [i64, i32, P]
    L.vco_group_values.restype = i32
    L.vco_group_values.argtypes = [P, i32, i64, i64, i32, i32, i32, P, P, P]
    L.vco_group_values_ex.restype = i32
    L.vco_group_values_ex.argtypes = [P, i32, i64, i64, i32, i32, i32, P, P, P, P, P]
    L.vco_k_mean.argtypes = [P, i32, i64, i64, i32, P, P]
    L.vco_quant_q.argtypes = [P, i32, i64, i64, i32, P, P]
    L.vco_quant_k.argtypes = [P, i32, i64, i64, i32, P, P, P, P]
    L.vco_quant_v_channel.argtypes = [P, i32, i64, i64, i32, P, P, P]
    L.vco_quant_v_smooth.argtypes = [P, i32, i64, i64, i32, P, i32, P, P, P]
    L.vco_attention.argtypes = [P, P, P, P, P, P, P, i32, i64, i64, i64, i32, f32, P, i64, P, P]
    L.vco_attention_control.argtypes = L.vco_attention.argtypes
    L.vco_attention_affine.argtypes = L.vco_attention.argtypes
    L.vco_attention_fp8.argtypes = [P, P, P, P, P, P, i64, i64, i64, i32, f32, P, i64, P, P, i32]
    L.vco_k_mean_f32.argtypes = [P, i32, i64, i64, i32, P]
    L.vco_quant_fp8_block.argtypes = [P, i32, i64, i64, i32, i32, P, P, P]
    L.vco_quant_q_rot.argtypes = L.vco_quant_q.argtypes
    L.vco_quant_k_rot.argtypes = L.vco_quant_k.argtypes
    L.vco_hadamard.argtypes = [P, i64, i32, P]
    L.vco_preprocess_qk.argtypes = [P, P, i32, i64, i64, i64, i32, i32, i32, P, P]


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- scalar maps

def expcast_codes(shifted) -> np.ndarray:
    x = _c(shifted, np.float32)
    y = np.empty(x.shape, np.uint8)
    lib().vco_expcast_codes(_ptr(x), _ptr(y), x.size)
    return y


def e4m3_encode(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint8)
    lib().vco_e4m3_encode_array(_ptr(x), _ptr(y), x.size)
    return y


def e4m3_decode(b) -> np.ndarray:
    b = _c(b, np.uint8)
    y = np.empty(b.shape, np.float32)
    lib().vco_e4m3_decode_array(_ptr(b), _ptr(y), b.size)
    return y


def exp2_rn(x: float) -> float:
    """Correctly rounded binary32 exp2 of a binary32 value."""
    return float(lib().vco_exp2_rn(float(np.float32(x))))


def fp8_exp2_codes(x) -> np.ndarray:
    """E4M3 bytes of the control path's probabilities exp2(x) (correctly rounded binary32)."""
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint8)
    lib().vco_fp8_exp2_codes(_ptr(x), _ptr(y), x.size)
    return y


def fp8_exp2_sweep(first_bits: int, n: int) -> np.ndarray:
    """fp8_exp2_codes of the binary32 values whose bits are first_bits .. first_bits + n - 1."""
    y = np.empty(n, np.uint8)
    lib().vco_fp8_exp2_sweep(first_bits, n, _ptr(y))
    return y


def cvt_u8(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint8)
    lib().vco_cvt_u8_array(_ptr(x), _ptr(y), x.size)
    return y


def tile_tree_sum(x) -> float:
    x = _c(x, np.float64)
    assert x.shape == (128,)
    return lib().vco_tile_tree_sum(_ptr(x))


def value_permutation(n: int) -> np.ndarray:
    """Sage's stored order within 16 tokens (reference vc_reference.py:14-17)."""
    i = np.arange(n)
    r = i % 16
    return (i // 16) * 16 + (r // 8) * 2 + ((r // 2) % 4) * 4 + r % 2


def linspace_ids(n: int, count: int) -> np.ndarray:
    ids = np.empty(count, np.int64)
    lib().vco_linspace_ids(n, count, _ptr(ids))
    return ids


# ---------------------------------------------------------------- preprocessing

def _shape4(x):
    x = np.asarray(x)
    if x.ndim != 4:
        raise ValueError("expected [B,H,N,D]")
    return x.shape


def group_values(v, clusters: int, iterations: int, dtype: str = "bfloat16", centers_in=None,
                 return_next: bool = False):
    """(perm, labels, centers of the final assignment[, centers_next]); centers_in warm-starts."""
    B, H, N, D = _shape4(v)
    v = _c(v, np.uint16)
    count = min(clusters, N)
    perm = np.empty((B, H, N), np.int64)
    labels = np.empty((B, H, N), np.int32)
    centers = np.empty((B, H, count, D), np.float32)
    nxt = np.empty((B, H, count, D), np.float32) if return_next else None
    cin = None if centers_in is None else _c(centers_in, np.float32)
    if cin is not None and cin.shape != (B, H, count, D):
        raise ValueError("centers_in must be [B,H,count,D]")
    rc = lib().vco_group_values_ex(_ptr(v), DTYPES[dtype], B * H, N, D, clusters, iterations, _ptr(cin),
                                   _ptr(perm), _ptr(labels), _ptr(centers), _ptr(nxt))
    if rc:
        raise ValueError("invalid clustering parameters")
    return (perm, labels, centers, nxt) if return_next else (perm, labels, centers)


def k_mean(k, perm=None, dtype: str = "bfloat16") -> np.ndarray:
    B, H, N, D = _shape4(k)
    k = _c(k, np.uint16)
    perm = None if perm is None else _c(perm, np.int64)
    km = np.empty((B, H, D), np.uint16)
    lib().vco_k_mean(_ptr(k), DTYPES[dtype], B * H, N, D, _ptr(perm), _ptr(km))
    return km


def quant_q(q, dtype: str = "bfloat16", rotate: bool = False):
    """Sage per-thread INT8 Q; rotate=True quantizes the Hadamard-rotated rows."""
    B, H, N, D = _shape4(q)
    q = _c(q, np.uint16)
    q8 = np.zeros((B, H, N, D), np.int8)
    qs = np.empty((B, H, (N + 63) // 64 * 32), np.float32)
    fn = lib().vco_quant_q_rot if rotate else lib().vco_quant_q
    fn(_ptr(q), DTYPES[dtype], B * H, N, D, _ptr(q8), _ptr(qs))
    return q8, qs


def quant_k(k, km=None, perm=None, dtype: str = "bfloat16", rotate: bool = False):
    """Sage per-thread INT8 K after centring; rotate=True rotates the centred rows first."""
    B, H, N, D = _shape4(k)
    k = _c(k, np.uint16)
    km = None if km is None else _c(km, np.uint16)
    perm = None if perm is None else _c(perm, np.int64)
    k8 = np.zeros((B, H, N, D), np.int8)
    ks = np.empty((B, H, (N + 127) // 128 * 4), np.float32)
    fn = lib().vco_quant_k_rot if rotate else lib().vco_quant_k
    fn(_ptr(k), DTYPES[dtype], B * H, N, D, _ptr(perm), _ptr(km), _ptr(k8), _ptr(ks))
    return k8, ks


def hadamard(x) -> np.ndarray:
    """Normalized Sylvester rotation of the last axis (core.py:79-92), zero padded to a
    power of two; binary32 butterflies in stride order."""
    x = np.ascontiguousarray(x, np.float32)
    D = x.shape[-1]
    W = 1 << (D - 1).bit_length()
    out = np.empty(x.shape[:-1] + (W,), np.float32)
    lib().vco_hadamard(_ptr(x), x.size // D, D, _ptr(out))
    return out


def preprocess_qk(q, k, *, k_smooth: bool, hadamard: bool, dtype: str = "float32"):
    """The reference's preprocess_qk (csrc/bindings.cpp:87-116): binary32 K centring over all
    keys and the normalized Q/K rotation. q, k: [B,H,N,D] arrays of the input dtype
    (float32 values, or uint16 bit patterns for float16/bfloat16)."""
    B, H, Nq, D = _shape4(q)
    Nk = np.asarray(k).shape[2]
    code = {"float16": 0, "bfloat16": 1, "float32": 2}[dtype]
    store = np.float32 if code == 2 else np.uint16
    q, k = _c(q, store), _c(k, store)
    W = (1 << (D - 1).bit_length()) if hadamard else D
    qo = np.empty((B, H, Nq, W), np.float32)
    ko = np.empty((B, H, Nk, W), np.float32)
    lib().vco_preprocess_qk(_ptr(q), _ptr(k), code, B * H, Nq, Nk, D, int(k_smooth), int(hadamard), _ptr(qo),
                            _ptr(ko))
    return qo, ko


def k_mean_f32(k, dtype: str = "bfloat16") -> np.ndarray:
    """vc27 K channel mean in binary32 (qk_fp8.cu:10-35)."""
    B, H, N, D = _shape4(k)
    km = np.empty((B, H, D), np.float32)
    lib().vco_k_mean_f32(_ptr(_c(k, np.uint16)), DTYPES[dtype], B * H, N, D, _ptr(km))
    return km


def quant_fp8_block(x, rows: int, mean=None, dtype: str = "bfloat16"):
    """Block E4M3 quantizer of vc27 (qk_fp8.cu:38-74): codes uint8 [B,H,N,D] and scales
    float32 [B,H,ceil(N/rows)]; mean (float32 [B,H,D]) centres first."""
    B, H, N, D = _shape4(x)
    codes = np.zeros((B, H, N, D), np.uint8)
    scales = np.empty((B, H, (N + rows - 1) // rows), np.float32)
    lib().vco_quant_fp8_block(_ptr(_c(x, np.uint16)), DTYPES[dtype], B * H, N, D, rows,
                              _ptr(None if mean is None else _c(mean, np.float32)), _ptr(codes), _ptr(scales))
    return codes, scales


def prepare_fp8(q, k, v, *, expcast=True, sm_scale=None, dtype: str = "bfloat16"):
    """State of the vc27 FP8 block-scaled QK path (vc_fp8.py:12-33): Q in 64-row E4M3
    blocks, K centred in binary32 and in 128-row blocks, V per-channel E4M3 (no smoothing)."""
    km = k_mean_f32(k, dtype)
    q8, qs = quant_fp8_block(q, 64, None, dtype)
    k8, ks = quant_fp8_block(k, 128, km, dtype)
    v8, vs = per_channel_fp8(v, None, dtype)
    D = np.asarray(q).shape[-1]
    return {"q": q8, "k": k8, "v": v8, "qs": qs, "ks": ks, "vs": vs, "means": None, "k_mean": km,
            "qk_format": "fp8_block", "expcast": bool(expcast), "block_values": False,
            "output_type": 1 if dtype == "bfloat16" else 0,
            "scale": D ** -0.5 if sm_scale is None else sm_scale, "permutation": None}


def per_thread_int8(q, k, km=None, perm=None, dtype: str = "bfloat16"):
    """Q per row-pair and K per key-set INT8 with FP32 scales (BLKQ=64, WARPQ=16, BLKK=128, WARPK=128)."""
    q8, qs = quant_q(q, dtype)
    k8, ks = quant_k(k, km, perm, dtype)
    return q8, qs, k8, ks


def per_channel_fp8(v, perm=None, dtype: str = "bfloat16"):
    """Smoothing-off V: LOGICAL payload [B,H,D,tiles*128] + per-channel scales [B,H,D]."""
    B, H, N, D = _shape4(v)
    v = _c(v, np.uint16)
    perm = None if perm is None else _c(perm, np.int64)
    npad = (N + 127) // 128 * 128
    v8 = np.empty((B, H, D, npad), np.uint8)
    vs = np.empty((B, H, D), np.float32)
    lib().vco_quant_v_channel(_ptr(v), DTYPES[dtype], B * H, N, D, _ptr(perm), _ptr(v8), _ptr(vs))
    return v8, vs


def prepare_values(v, perm=None, channel_scale: bool = True, dtype: str = "bfloat16"):
    """Smoothing-on V: LOGICAL payload, scales ([B,H,D] or [B,H,tiles,D]), fp16 means bits [B,H,tiles,D]."""
    B, H, N, D = _shape4(v)
    v = _c(v, np.uint16)
    perm = None if perm is None else _c(perm, np.int64)
    tiles = (N + 127) // 128
    v8 = np.empty((B, H, D, tiles * 128), np.uint8)
    vs = np.empty((B, H, D) if channel_scale else (B, H, tiles, D), np.float32)
    means = np.empty((B, H, tiles, D), np.uint16)
    lib().vco_quant_v_smooth(_ptr(v), DTYPES[dtype], B * H, N, D, _ptr(perm), int(channel_scale),
                             _ptr(v8), _ptr(vs), _ptr(means))
    return v8, vs, means


def prepare(q, k, v, *, expcast=True, v_smooth=True, clusters=8, iterations=2, sm_scale=None,
            v_scale_mode="channel", dtype="bfloat16", qk_hadamard=False, permutation=None):
    """State dict of the sageattn_vc contract (reference vc.py:141-170); v is LOGICAL.

    expcast only selects the probability path of ``reference``; the payloads are the same.
    qk_hadamard rotates Q and the centred K before the INT8 quantizer. permutation (int64
    [B,H,N]) replaces the grouping: K and V are gathered by it whether or not smoothing is
    on, as vc_attention does with a cached layout (src/vc_attention/core.py:305-310).
    """
    perm = None
    if permutation is not None:
        perm = np.ascontiguousarray(permutation, dtype=np.int64)
    elif v_smooth:
        perm, _, _ = group_values(v, clusters, iterations, dtype)
    km = k_mean(k, perm, dtype)
    q8, qs = quant_q(q, dtype, rotate=qk_hadamard)
    k8, ks = quant_k(k, km, perm, dtype, rotate=qk_hadamard)
    if v_smooth:
        v8, vs, means = prepare_values(v, perm, v_scale_mode == "channel", dtype)
    else:
        v8, vs = per_channel_fp8(v, perm, dtype)
        means = None
    D = np.asarray(q).shape[-1]
    return {"q": q8, "k": k8, "v": v8, "qs": qs, "ks": ks, "vs": vs, "means": means, "km": km,
            "expcast": bool(expcast), "block_values": v_smooth, "output_type": 1 if dtype == "bfloat16" else 0,
            "scale": D ** -0.5 if sm_scale is None else sm_scale, "permutation": perm}


def reference(state, query_indices=None, return_codes=False, affine=False):
    """Decoded-payload oracle (vc_reference.py:20-91) with the exact P bytes.

    state["expcast"] False selects the Sage FP8 control path (vc_reference.py:58-66):
    the bytes are then E4M3(exp2(...)) and the mass is the unrounded exp2 sum.
    affine=True selects the folded ExpCast encode of the reference's default kernel modes
    (vc12..vc15, "optimized"; sal/csrc/vc/vc_math.cuh:16-111), which the reference only
    uses without block values.
    Returns float32 [B,H,len(ids),D] (and uint8 codes [B,H,len(ids),tiles*128]).
    """
    q8, k8, v8 = state["q"], state["k"], state["v"]
    B, H, Nq, D = q8.shape
    Nk = k8.shape[2]
    tiles = (Nk + 127) // 128
    ids = np.arange(Nq, dtype=np.int64) if query_indices is None else np.asarray(query_indices, np.int64)
    if ids.size == 0:
        raise ValueError("Reference requires nonempty queries")
    vs = state["vs"]
    means = state.get("means")
    block_scale = int(means is not None and vs is not None and vs.ndim == 4)
    out = np.empty((B, H, ids.size, D), np.float32)
    codes = np.empty((B, H, ids.size, tiles * 128), np.uint8) if return_codes else None
    if state.get("qk_format", "int8") == "fp8_block":
        if means is not None or vs is None or vs.ndim != 3:
            raise ValueError("the FP8 block QK path has no block values")
        mode = 0 if not state.get("expcast", True) else (2 if affine else 1)
        lib().vco_attention_fp8(_ptr(_c(q8, np.uint8)), _ptr(_c(k8, np.uint8)), _ptr(_c(v8, np.uint8)),
                                _ptr(_c(state["qs"], np.float32)), _ptr(_c(state["ks"], np.float32)),
                                _ptr(_c(vs, np.float32)), B * H, Nq, Nk, D, float(np.float32(state["scale"])),
                                _ptr(ids), ids.size, _ptr(out), _ptr(codes), mode)
        return (out, codes) if return_codes else out
    if affine and (not state.get("expcast", True) or means is not None):
        raise ValueError("the folded ExpCast encode applies to ExpCast without block values")
    fn = (lib().vco_attention_control if not state.get("expcast", True)
          else lib().vco_attention_affine if affine else lib().vco_attention)
    fn(_ptr(_c(q8, np.int8)), _ptr(_c(k8, np.int8)), _ptr(_c(v8, np.uint8)),
       _ptr(_c(state["qs"], np.float32)), _ptr(_c(state["ks"], np.float32)),
       _ptr(None if vs is None else _c(vs, np.float32)),
       _ptr(None if means is None else _c(means, np.uint16)), block_scale,
       B * H, Nq, Nk, D, float(np.float32(state["scale"])), _ptr(ids), ids.size,
       _ptr(out), _ptr(codes))
    return (out, codes) if return_codes else out


def query_indices(n: int, count: int = 128) -> np.ndarray:
    """Evenly spaced sample rows i*(n-1)//(count-1) (reference scripts/benchmark_cuda.py:224-228)."""
    if n <= count:
        return np.arange(n, dtype=np.int64)
    return np.array([i * (n - 1) // (count - 1) for i in range(count)], np.int64)
