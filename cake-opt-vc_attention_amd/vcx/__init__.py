"""ctypes binding of libvcx.so (include/vcx.h) for PyTorch-ROCm tensors.

This module is the only Python code that touches the native library. It
allocates outputs and workspaces with torch (so the caching allocator and the
current HIP stream semantics hold), passes raw pointers, shapes and strides to
the C ABI, and turns nonzero status codes into exceptions. There is no CPU or
eager fallback: a missing or stale library raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import functools
import itertools
from pathlib import Path

import torch

ABI_VERSION = 3
LIB_PATH = Path(__file__).resolve().parents[1] / "lib" / "libvcx.so"

_OK, _EINVAL, _EUNSUPPORTED, _EHIP = 0, 1, 2, 3
NOALLOC_SCRATCH_BYTES = 32 << 20  # VCX_NOALLOC_SCRATCH_BYTES
WS_PREPARE_QK, WS_PREPARE_V, WS_GROUP, WS_PREPROCESS_QK = 1, 2, 3, 4
_DTYPE = {torch.float16: 0, torch.bfloat16: 1}
_PRE_DTYPE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
_lib = None


class VcxError(RuntimeError):
    """A libvcx call returned an error status."""


def _declare(L):
    P, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
    L.vcx_abi_version.restype = i32
    L.vcx_clock_probe.restype = i32
    L.vcx_clock_probe.argtypes = [i64, P, ctypes.POINTER(ctypes.c_int), P]
    L.vcx_abi_version.argtypes = []
    L.vcx_last_error.restype = ctypes.c_char_p
    L.vcx_last_error.argtypes = []
    L.vcx_value_token.restype = i32
    L.vcx_value_token.argtypes = [i32]
    L.vcx_workspace_bytes.restype = i32
    L.vcx_workspace_bytes.argtypes = [i32, i64, i64, i64, i64, i32, i32, ctypes.POINTER(ctypes.c_size_t)]
    L.vcx_group_values.restype = i32
    L.vcx_group_values.argtypes = [P, i32, i64, i64, i64, i64, i64, i64, i64, i32, i32, i32, P, P, P, P, P, P,
                                   ctypes.c_size_t, P]
    L.vcx_prepare_qk_int8.restype = i32
    L.vcx_prepare_qk_int8.argtypes = [P, P, i32, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64,
                                      P, P, P, P, P, P, P, ctypes.c_size_t, P]
    L.vcx_prepare_qk_int8_noalloc.restype = i32
    L.vcx_prepare_qk_int8_noalloc.argtypes = [P, P, i32, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64,
                                              P, P, P, P, P, P, P]
    L.vcx_prepare_qk_int8_rotated.restype = i32
    L.vcx_prepare_qk_int8_rotated.argtypes = L.vcx_prepare_qk_int8.argtypes
    L.vcx_preprocess_qk.restype = i32
    L.vcx_preprocess_qk.argtypes = [P, P, i32, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i32, i32,
                                    P, P, P, ctypes.c_size_t, P]
    L.vcx_prepare_qk_fp8.restype = i32
    L.vcx_prepare_qk_fp8.argtypes = [P, P, i32, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64,
                                     P, P, P, P, P, P, ctypes.c_size_t, P]
    L.vcx_prepare_v_fp8.restype = i32
    L.vcx_prepare_v_fp8.argtypes = [P, i32, i64, i64, i64, i64, i64, i64, i64, P, i32, i32, P, P, P, P,
                                    ctypes.c_size_t, P]
    L.vcx_attention_fwd.restype = i32
    L.vcx_attention_fwd.argtypes = [P, P, P, P, P, P, P, i64, i64, i64, i64, i64, i32, i32, i32, f32, i32,
                                    P, i64, i64, i64, P, i64, i64, P]
    L.vcx_attention_fwd_fp8.restype = i32
    L.vcx_attention_fwd_fp8.argtypes = [P, P, P, P, P, P, i64, i64, i64, i64, i64, i32, f32, i32,
                                        P, i64, i64, i64, P, i64, i64, P]
    L.vcx_expcast_codes.restype = i32
    L.vcx_expcast_codes.argtypes = [P, P, i64, P]
    L.vcx_fp8_exp2_codes.restype = i32
    L.vcx_fp8_exp2_codes.argtypes = [P, P, i64, i32, P]
    L.vcx_convert_probe.restype = i32
    L.vcx_convert_probe.argtypes = [P, P, P, i64, P]
    L.vcx_kernel_resources.restype = i32
    L.vcx_kernel_resources.argtypes = [i64, i32, ctypes.POINTER(ctypes.c_int64)]
    L.vcx_kernel_resources_mode.restype = i32
    L.vcx_kernel_resources_mode.argtypes = [i64, i32, i32, i32, ctypes.POINTER(ctypes.c_int64)]
    L.vcx_kernel_resources_fp8.restype = i32
    L.vcx_kernel_resources_fp8.argtypes = [i64, i32, ctypes.POINTER(ctypes.c_int64)]


EXPORTED = ("vcx_abi_version", "vcx_last_error", "vcx_value_token", "vcx_workspace_bytes",
            "vcx_group_values", "vcx_prepare_qk_int8", "vcx_prepare_qk_int8_noalloc", "vcx_prepare_qk_int8_rotated",
            "vcx_preprocess_qk",
            "vcx_prepare_qk_fp8", "vcx_prepare_v_fp8", "vcx_attention_fwd", "vcx_attention_fwd_fp8",
            "vcx_expcast_codes", "vcx_fp8_exp2_codes", "vcx_convert_probe", "vcx_kernel_resources", "vcx_kernel_resources_mode",
            "vcx_kernel_resources_fp8",
            "vcx_clock_probe")


def _device_call(fn):
    """no_grad, with the device of the first tensor argument made current for the call: the
    library launches on the current HIP device, on a stream of that device."""

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        t = next((a for a in itertools.chain(args, kwargs.values()) if isinstance(a, torch.Tensor)), None)
        with torch.no_grad():
            if t is not None and t.device.type == "cuda":
                with torch.cuda.device(t.device):
                    return fn(*args, **kwargs)
            return fn(*args, **kwargs)

    return wrapper


def lib():
    """Load libvcx.so once and check its ABI version (raises RuntimeError, never falls back)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"libvcx.so is missing at {LIB_PATH}; build it with "
                               "python cake-opt-vc_attention_amd/build.py. No fallback was used.")
        L = ctypes.CDLL(str(LIB_PATH))
        _declare(L)
        if L.vcx_abi_version() != ABI_VERSION:
            raise RuntimeError("Stale libvcx.so (ABI %d, expected %d): rebuild it" % (L.vcx_abi_version(), ABI_VERSION))
        _lib = L
    return _lib


def _check(rc: int, what: str):
    if rc == _OK:
        return
    msg = lib().vcx_last_error().decode(errors="replace")
    if rc == _EUNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise VcxError(f"{what}: {msg}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_device(*tensors):
    dev = tensors[0].device
    if dev.type != "cuda":
        raise VcxError("libvcx requires GPU (HIP) tensors; no CPU fallback")
    for t in tensors:
        if t is not None and t.device != dev:
            raise VcxError("all tensors must be on the same device")
    return dev


def _strides4(x):
    if x.dim() != 4 or x.stride(3) != 1:
        raise VcxError("expected [B,H,N,D] with a contiguous last dimension")
    return x.stride(0), x.stride(1), x.stride(2)


def _check_qk_pair(q, k):
    """Q and K must agree in batch, heads and head dim: the C ABI takes one B/H/D for both."""
    if q.dim() != 4 or k.dim() != 4:
        raise VcxError("Q/K must be [B,H,N,D]")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[3] != k.shape[3]:
        raise VcxError(f"Q {tuple(q.shape)} and K {tuple(k.shape)} must match in batch, heads and head dim")
    if q.numel() == 0 or k.numel() == 0:
        raise VcxError("Q/K must be nonempty")


def _output(out, shape, dtype, device):
    """The caller's output buffer (checked against what the kernel writes) or a new one."""
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    if tuple(out.shape) != tuple(shape) or out.dtype != dtype or out.device != device:
        raise VcxError(f"out must be {dtype} {tuple(shape)} on {device}; got {out.dtype} "
                       f"{tuple(out.shape)} on {out.device}")
    return out


def workspace_bytes(op: int, B: int, H: int, N: int, D: int, smooth: bool = False, clusters: int = 8) -> int:
    out = ctypes.c_size_t(0)
    _check(lib().vcx_workspace_bytes(op, B, H, N, D, int(smooth), clusters, ctypes.byref(out)),
           "vcx_workspace_bytes")
    return out.value


def _workspace(nbytes: int, device):
    # torch allocations are at least 256-byte aligned on ROCm.
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


def value_token():
    """Token offset stored at each byte position of a 128-token V tile (storage order)."""
    return [lib().vcx_value_token(p) for p in range(128)]


def value_position_index(device=None):
    """Index tensor that maps storage order -> logical token order inside each tile."""
    tok = value_token()
    pos = [0] * 128
    for p, t in enumerate(tok):
        pos[t] = p
    return torch.tensor(pos, dtype=torch.long, device=device)


def abi_version() -> int:
    return lib().vcx_abi_version()


# ---------------------------------------------------------------- preprocessing

GROUP_AUTO, GROUP_GENERAL = 0, 1


@_device_call
def group_values(v, clusters: int, iterations: int, debug: bool = False, *, legacy: bool = False,
                 centers=None, return_centers: bool = False):
    """Lloyd grouping of V tokens -> int64 permutation [B,H,N].

    debug=True also returns int32 labels and the final assignment's fp32 centers
    [B,H,count,D]; return_centers=True appends centers_next, the update of the final labels
    (pass it back as `centers` to warm-start the next call). legacy=True runs the general
    schedule for every count (the reference's group_values_legacy); otherwise counts above 8
    take it and the rest the fused one. Results are identical between the two.
    """
    if v.dtype not in _DTYPE:
        raise VcxError("grouping requires float16/bfloat16 V")
    if v.dim() != 4:
        raise VcxError("V must be [B,H,N,D]")
    B, H, N, D = v.shape
    count = min(clusters, N)
    if centers is not None and (centers.dtype != torch.float32 or tuple(centers.shape) != (B, H, count, D)
                                or not centers.is_contiguous()):
        raise VcxError(f"centers must be contiguous float32 {(B, H, count, D)}")
    dev = _require_device(v, centers)
    sb, sh, sn = _strides4(v)
    perm = torch.empty((B, H, N), dtype=torch.int64, device=dev)
    labels = torch.empty((B, H, N), dtype=torch.int32, device=dev) if debug else None
    cen = torch.empty((B, H, count, D), dtype=torch.float32, device=dev) if debug else None
    nxt = torch.empty((B, H, count, D), dtype=torch.float32, device=dev) if return_centers else None
    ws = _workspace(workspace_bytes(WS_GROUP, B, H, N, D, clusters=clusters), dev)
    _check(lib().vcx_group_values(_ptr(v), _DTYPE[v.dtype], B, H, N, D, sb, sh, sn, clusters, iterations,
                                  GROUP_GENERAL if legacy else GROUP_AUTO, _ptr(centers), _ptr(perm),
                                  _ptr(labels), _ptr(cen), _ptr(nxt), _ptr(ws), ws.numel(), _stream(dev)),
           "vcx_group_values")
    out = (perm, labels, cen) if debug else (perm,)
    if return_centers:
        out = out + (nxt,)
    return out if len(out) > 1 else perm


@_device_call
def prepare_qk(q, k, perm=None, hadamard: bool = False):
    """INT8 Q/K with Sage per-thread scales after K centring: (q8, qs, k8, ks, km).
    hadamard=True rotates Q and the centred K (normalized Sylvester transform) first."""
    if q.dtype not in _DTYPE or k.dtype != q.dtype:
        raise VcxError("Q/K require matching float16/bfloat16")
    _check_qk_pair(q, k)
    dev = _require_device(q, k, perm)
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    qsb, qsh, qsn = _strides4(q)
    ksb, ksh, ksn = _strides4(k)
    if perm is not None and (perm.dtype != torch.int64 or tuple(perm.shape) != (B, H, Nk) or not perm.is_contiguous()):
        raise VcxError("perm must be contiguous int64 [B,H,Nk]")
    q8 = torch.empty((B, H, Nq, D), dtype=torch.int8, device=dev)
    k8 = torch.empty((B, H, Nk, D), dtype=torch.int8, device=dev)
    qs = torch.empty((B, H, (Nq + 63) // 64 * 32), dtype=torch.float32, device=dev)
    ks = torch.empty((B, H, (Nk + 127) // 128 * 4), dtype=torch.float32, device=dev)
    km = torch.empty((B, H, 1, D), dtype=q.dtype, device=dev)
    ws = _workspace(workspace_bytes(WS_PREPARE_QK, B, H, Nk, D), dev)
    name = "vcx_prepare_qk_int8_rotated" if hadamard else "vcx_prepare_qk_int8"
    _check(getattr(lib(), name)(_ptr(q), _ptr(k), _DTYPE[q.dtype], B, H, Nq, Nk, D, qsb, qsh, qsn,
                                ksb, ksh, ksn, _ptr(perm), _ptr(q8), _ptr(qs), _ptr(k8), _ptr(ks), _ptr(km),
                                _ptr(ws), ws.numel(), _stream(dev)), name)
    return q8, qs, k8, ks, km


@_device_call
def preprocess_qk(q, k, k_smooth: bool, hadamard: bool):
    """Binary32 post-RoPE Q/K preprocessing (the reference's preprocess_qk): K centred by its
    channel mean when k_smooth, Q and K rotated by the normalized Sylvester-Hadamard transform
    (zero padded to a power of two) when hadamard. fp16/bf16/fp32 [B,H,N,D], D <= 128."""
    dev = _require_device(q, k)
    if q.dim() != 4 or k.dim() != 4 or q.numel() == 0 or k.numel() == 0:
        raise VcxError("Expected nonempty [B,H,N,D]")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[3] != k.shape[3]:
        raise VcxError("Q/K shapes must match")
    if q.dtype not in _PRE_DTYPE or k.dtype != q.dtype:
        raise VcxError("Q/K require one of float16/bfloat16/float32")
    if q.stride(-1) != 1 or k.stride(-1) != 1:
        q, k = q.contiguous(), k.contiguous()
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    W = (1 << (D - 1).bit_length()) if hadamard else D
    qo = torch.empty((B, H, Nq, W), dtype=torch.float32, device=dev)
    ko = torch.empty((B, H, Nk, W), dtype=torch.float32, device=dev)
    ws = _workspace(workspace_bytes(WS_PREPROCESS_QK, B, H, Nk, D), dev) if k_smooth else None
    _check(lib().vcx_preprocess_qk(_ptr(q), _ptr(k), _PRE_DTYPE[q.dtype], B, H, Nq, Nk, D, *q.stride()[:3],
                                   *k.stride()[:3], int(k_smooth), int(hadamard), _ptr(qo), _ptr(ko), _ptr(ws),
                                   0 if ws is None else ws.numel(), _stream(dev)), "vcx_preprocess_qk")
    return qo, ko


@_device_call
def prepare_qk_fp8(q, k):
    """Block-scaled E4M3 Q/K (Q 64-row blocks, centred K 128-row blocks):
    (q8 uint8 [B,H,Nq,D], qs [B,H,ceil(Nq/64)], k8 uint8 [B,H,Nk,D], ks [B,H,ceil(Nk/128)],
    km fp32 [B,H,D])."""
    if q.dtype not in _DTYPE or k.dtype != q.dtype:
        raise VcxError("Q/K require matching float16/bfloat16")
    _check_qk_pair(q, k)
    dev = _require_device(q, k)
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    qsb, qsh, qsn = _strides4(q)
    ksb, ksh, ksn = _strides4(k)
    q8 = torch.empty((B, H, Nq, D), dtype=torch.uint8, device=dev)
    k8 = torch.empty((B, H, Nk, D), dtype=torch.uint8, device=dev)
    qs = torch.empty((B, H, (Nq + 63) // 64), dtype=torch.float32, device=dev)
    ks = torch.empty((B, H, (Nk + 127) // 128), dtype=torch.float32, device=dev)
    km = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    ws = _workspace(workspace_bytes(WS_PREPARE_QK, B, H, Nk, D), dev)
    _check(lib().vcx_prepare_qk_fp8(_ptr(q), _ptr(k), _DTYPE[q.dtype], B, H, Nq, Nk, D, qsb, qsh, qsn,
                                    ksb, ksh, ksn, _ptr(q8), _ptr(qs), _ptr(k8), _ptr(ks), _ptr(km),
                                    _ptr(ws), ws.numel(), _stream(dev)), "vcx_prepare_qk_fp8")
    return q8, qs, k8, ks, km


@_device_call
def prepare_v(v, perm=None, smooth: bool = False, channel_scale: bool = True):
    """E4M3 V in storage order: (v8 [B,H,D,tiles*128], vs, means or empty)."""
    dev = _require_device(v, perm)
    if v.dtype not in _DTYPE:
        raise VcxError("V requires float16/bfloat16")
    B, H, N, D = v.shape
    sb, sh, sn = _strides4(v)
    if perm is not None and (perm.dtype != torch.int64 or tuple(perm.shape) != (B, H, N) or not perm.is_contiguous()):
        raise VcxError("perm must be contiguous int64 [B,H,N]")
    tiles = (N + 127) // 128
    v8 = torch.empty((B, H, D, tiles * 128), dtype=torch.float8_e4m3fn, device=dev)
    if smooth:
        vs = torch.empty((B, H, D) if channel_scale else (B, H, tiles, D), dtype=torch.float32, device=dev)
        means = torch.empty((B, H, tiles, D), dtype=torch.float16, device=dev)
    else:
        vs = torch.empty((B, H, D), dtype=torch.float32, device=dev)
        means = torch.empty(0, dtype=torch.float16, device=dev)
    ws = _workspace(workspace_bytes(WS_PREPARE_V, B, H, N, D, smooth), dev)
    _check(lib().vcx_prepare_v_fp8(_ptr(v), _DTYPE[v.dtype], B, H, N, D, sb, sh, sn, _ptr(perm), int(smooth),
                                   int(channel_scale), _ptr(v8), _ptr(vs), _ptr(means) if smooth else None,
                                   _ptr(ws), ws.numel(), _stream(dev)), "vcx_prepare_v_fp8")
    return v8, vs, means


# ---------------------------------------------------------------- attention

@_device_call
def forward(q8, k8, v8, qs, ks, vs, means, expcast: bool, block_values: bool, output_type: int, scale: float,
            *, channel_scale: bool = True, affine: bool = False, out=None, p_rows=None):
    """Fused attention on prepared payloads -> out [B,H,Nq,D] (fp16 if output_type == 0 else bf16).

    expcast=False runs the Sage FP8 control probabilities. affine=True (ExpCast without
    block values only) selects the folded encode of the reference's default kernel modes
    (vc12..vc15, "optimized"); affine=False the unfused encode (vc4..vc11 and every
    block-value launch).
    p_rows=(begin, end) additionally returns the E4M3 P bytes of those query rows
    (uint8 [B,H,end-begin,tiles*128], logical key order) from the diagnostic variant.
    """
    if affine and (not expcast or block_values):
        raise VcxError("the folded ExpCast encode applies to ExpCast without block values")
    if q8.dim() != 4:
        raise VcxError("q must be [B,H,Nq,D]")
    B, H, Nq, D = q8.shape
    Nk = k8.shape[2]
    tiles = (Nk + 127) // 128
    for name, t, dt in (("q", q8, torch.int8), ("k", k8, torch.int8), ("qs", qs, torch.float32),
                        ("ks", ks, torch.float32), ("vs", vs, torch.float32)):
        if t.dtype != dt or not t.is_contiguous():
            raise VcxError(f"{name} must be contiguous {dt}")
    if v8.dtype not in (torch.float8_e4m3fn, torch.uint8) or not v8.is_contiguous():
        raise VcxError("v must be contiguous float8_e4m3fn")
    if tuple(k8.shape) != (B, H, Nk, D) or tuple(v8.shape) != (B, H, D, tiles * 128):
        raise VcxError("K/V payload shapes do not match Q")
    if tuple(qs.shape) != (B, H, (Nq + 63) // 64 * 32) or tuple(ks.shape) != (B, H, tiles * 4):
        raise VcxError("qs/ks shapes do not match the payloads")
    if block_values:
        if means is None or means.dtype != torch.float16 or tuple(means.shape) != (B, H, tiles, D) \
                or not means.is_contiguous():
            raise VcxError("means must be contiguous float16 [B,H,tiles,D]")
    vs_shape = (B, H, D) if (channel_scale or not block_values) else (B, H, tiles, D)
    if tuple(vs.shape) != vs_shape:
        raise VcxError(f"vs must have shape {vs_shape}")
    out_dtype = torch.float16 if output_type == 0 else torch.bfloat16
    out = _output(out, (B, H, Nq, D), out_dtype, q8.device)
    dev = _require_device(q8, k8, v8, qs, ks, vs, means if block_values else None, out)
    osb, osh, osn = _strides4(out)
    pd = None
    r0 = r1 = 0
    if p_rows is not None:
        r0, r1 = int(p_rows[0]), int(p_rows[1])
        pd = torch.zeros((B, H, max(r1 - r0, 0), tiles * 128), dtype=torch.uint8, device=dev)
    _check(lib().vcx_attention_fwd(_ptr(q8), _ptr(k8), _ptr(v8), _ptr(qs), _ptr(ks), _ptr(vs),
                                   _ptr(means) if block_values else None, B, H, Nq, Nk, D,
                                   (2 if affine else 1) if expcast else 0,
                                   int(block_values), int(channel_scale), float(scale), 1 if output_type else 0,
                                   _ptr(out), osb, osh, osn, _ptr(pd), r0, r1, _stream(dev)),
           "vcx_attention_fwd")
    return (out, pd) if p_rows is not None else out


@_device_call
def forward_fp8(q8, k8, v8, qs, ks, vs, expcast: bool, output_type: int, scale: float,
                *, affine: bool = True, out=None, p_rows=None):
    """Fused attention on block-scaled FP8 Q/K payloads (vcx.prepare_qk_fp8) and the
    per-channel V payload (vcx.prepare_v) -> out [B,H,Nq,D].

    expcast=True folds the ExpCast encode (affine=True, the reference's FP8 kernel) or
    runs the unfused encode (affine=False); expcast=False runs the Sage FP8 control
    probabilities. p_rows as in forward().
    """
    if q8.dim() != 4:
        raise VcxError("q must be [B,H,Nq,D]")
    B, H, Nq, D = q8.shape
    Nk = k8.shape[2]
    tiles = (Nk + 127) // 128
    for name, t in (("q", q8), ("k", k8), ("v", v8)):
        if t.dtype not in (torch.float8_e4m3fn, torch.uint8) or not t.is_contiguous():
            raise VcxError(f"{name} must be contiguous float8_e4m3fn")
    for name, t in (("qs", qs), ("ks", ks), ("vs", vs)):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise VcxError(f"{name} must be contiguous float32")
    if tuple(k8.shape) != (B, H, Nk, D) or tuple(v8.shape) != (B, H, D, tiles * 128):
        raise VcxError("K/V payload shapes do not match Q")
    if tuple(qs.shape) != (B, H, (Nq + 63) // 64) or tuple(ks.shape) != (B, H, tiles) \
            or tuple(vs.shape) != (B, H, D):
        raise VcxError("Incorrect FP8 block scales")
    out_dtype = torch.float16 if output_type == 0 else torch.bfloat16
    out = _output(out, (B, H, Nq, D), out_dtype, q8.device)
    dev = _require_device(q8, k8, v8, qs, ks, vs, out)
    osb, osh, osn = _strides4(out)
    pd = None
    r0 = r1 = 0
    if p_rows is not None:
        r0, r1 = int(p_rows[0]), int(p_rows[1])
        pd = torch.zeros((B, H, max(r1 - r0, 0), tiles * 128), dtype=torch.uint8, device=dev)
    _check(lib().vcx_attention_fwd_fp8(_ptr(q8), _ptr(k8), _ptr(v8), _ptr(qs), _ptr(ks), _ptr(vs), B, H, Nq, Nk,
                                       D, (2 if affine else 1) if expcast else 0, float(scale),
                                       1 if output_type else 0, _ptr(out), osb, osh, osn, _ptr(pd), r0, r1,
                                       _stream(dev)),
           "vcx_attention_fwd_fp8")
    return (out, pd) if p_rows is not None else out


@_device_call
def expcast_codes(x):
    dev = _require_device(x)
    x = x.float().contiguous()
    y = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    _check(lib().vcx_expcast_codes(_ptr(x), _ptr(y), x.numel(), _stream(dev)), "vcx_expcast_codes")
    return y


@_device_call
def fp8_exp2_codes(x, last_tile: bool = False):
    """E4M3 bytes of the control path's probabilities exp2(x), from the fused kernel's device
    code (last_tile: the saturating window form, which the kernel runs on every tile; else
    the 64-bit pair form; the bytes are the same)."""
    dev = _require_device(x)
    x = x.float().contiguous()
    y = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    _check(lib().vcx_fp8_exp2_codes(_ptr(x), _ptr(y), x.numel(), int(last_tile), _stream(dev)),
           "vcx_fp8_exp2_codes")
    return y


@_device_call
def convert_probe(x):
    dev = _require_device(x)
    x = x.float().contiguous()
    u8 = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    f8 = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    _check(lib().vcx_convert_probe(_ptr(x), _ptr(u8), _ptr(f8), x.numel(), _stream(dev)), "vcx_convert_probe")
    return u8, f8


CLOCK_PROBE_BLOCKS = 8


class ClockProbe:
    """Engine-clock reading (one wave per XCD) launched on the current stream of `device`;
    ghz() and ghz_per_block() synchronize the device."""

    def __init__(self, window_us: int, device=None):
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.ticks = torch.zeros(2 * CLOCK_PROBE_BLOCKS, dtype=torch.int64, device=dev)
        khz = ctypes.c_int(0)
        with torch.cuda.device(dev):
            _check(lib().vcx_clock_probe(int(window_us), _ptr(self.ticks), ctypes.byref(khz), _stream(dev)),
                   "vcx_clock_probe")
        self.wall_khz = khz.value

    def ghz_per_block(self) -> list:
        torch.cuda.synchronize(self.ticks.device)
        t = [int(x) for x in self.ticks.cpu()]
        return [t[2 * i] / t[2 * i + 1] * self.wall_khz / 1e6 for i in range(CLOCK_PROBE_BLOCKS)]

    def ghz(self) -> float:
        """Mean engine clock over the probe blocks, GHz."""
        g = self.ghz_per_block()
        return sum(g) / len(g)


def clock_probe(window_us: int, device=None) -> ClockProbe:
    """Launch one wave that counts engine-clock ticks against the constant-rate real-time
    counter for `window_us` microseconds (asynchronous; read the result with .ghz())."""
    return ClockProbe(window_us, device)


def kernel_resources_mode(D: int, value_mode: int, expcast: int, output_type: int = 1) -> dict:
    """Compiled resources of the fused kernel one launch mode runs (value_mode 0: no block
    values, 1: block values with channel scales, 2: per-block scales; expcast 0 control,
    1 unfused ExpCast, 2 folded), in the reference's key names (vc_sm90.cu:786-797)."""
    arr = (ctypes.c_int64 * 7)()
    _check(lib().vcx_kernel_resources_mode(D, value_mode, expcast, 1 if output_type else 0, arr),
           "vcx_kernel_resources_mode")
    return {"registers_per_thread": arr[0], "local_bytes_per_thread": arr[5], "static_shared_bytes": arr[2],
            "dynamic_shared_bytes": arr[3], "threads_per_block": arr[4], "predicted_active_blocks_per_sm": arr[6]}


def kernel_resources(D: int = 128, block_values: bool = False, *, qk_fp8: bool = False,
                     expcast: bool = True) -> dict:
    arr = (ctypes.c_int64 * 6)()
    if qk_fp8:
        _check(lib().vcx_kernel_resources_fp8(D, int(expcast), arr), "vcx_kernel_resources_fp8")
    else:
        _check(lib().vcx_kernel_resources(D, int(block_values), arr), "vcx_kernel_resources")
    return {"vgprs": arr[0], "agprs": arr[1], "static_lds_bytes": arr[2], "dynamic_lds_bytes": arr[3],
            "threads_per_block": arr[4], "scratch_bytes_per_lane": arr[5]}
