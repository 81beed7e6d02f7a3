"""Block-scaled FP8 QK + FP8 PV attention on MI355X (gfx950): the reference's
experimental vc27 path (third_party/sageattention_local/sageattention_local/vc_fp8.py).

Noncausal MHA, FP16/BF16 input and output, D64/D128. Q is quantized to E4M3 in
64-row blocks and K, after centring by its binary32 channel mean, in 128-row
blocks, each block with one FP32 scale; V is the per-channel E4M3 payload of
the INT8 path without smoothing. No QK rotation and no V smoothing. With
``expcast=True`` the probabilities are the folded ExpCast encode (as the
reference's FP8 kernel), otherwise the Sage FP8 control path.

Same functions, arguments and ValueError checks as the reference module, with
these deliberate differences:
* gfx950 instead of Hopper; any current HIP stream is accepted;
* the V payload is in the gfx950 tile storage order (``vcx.value_token``);
* Q/K payloads are returned as uint8 E4M3 bytes.
All native work runs in libvcx.so through :mod:`vcx`; there is no CPU fallback.
"""
import torch

import vcx

from .vc import _check_scale, _extension, _require_gfx950, validate_inputs


@torch.no_grad()
def prepare(q, k, v, *, expcast=True, sm_scale=None):
    """HND preparation (reference vc_fp8.py:12-33) on the current stream."""
    ext = _extension()
    q8, qs, k8, ks, km = ext.prepare_qk_fp8(q, k)
    v8, vs, means = ext.prepare_v(v, None, smooth=False, channel_scale=True)
    return {"q": q8, "k": k8, "v": v8, "qs": qs, "ks": ks, "vs": vs,
            "means": torch.empty(0, device=q.device, dtype=torch.float16),
            "k_mean": km, "qk_format": "fp8_block", "expcast": expcast,
            "block_values": False, "output_type": 0 if q.dtype == torch.float16 else 1,
            "scale": q.shape[-1] ** -0.5 if sm_scale is None else sm_scale, "permutation": None,
            "v_layout": "gfx950_tile128"}


@torch.no_grad()
def forward_prepared(state, *, out=None):
    """Fused FP8 kernel on a prepared state (reference vc_fp8.py:36-42)."""
    if state.get("qk_format") != "fp8_block" or state.get("block_values", False):
        raise ValueError("Expected FP8 block QK without V smoothing")
    return _extension().forward_fp8(*(state[key] for key in
                                      ("q", "k", "v", "qs", "ks", "vs", "expcast", "output_type", "scale")),
                                    out=out)


@torch.no_grad()
def sageattn_vc_fp8(q, k, v, tensor_layout="HND", is_causal=False, sm_scale=None, return_lse=False, *,
                    expcast=True):
    """Fresh block FP8 quantization and one fused attention launch (reference vc_fp8.py:45-62)."""
    validate_inputs(q, k, v, tensor_layout, is_causal, return_lse, expcast, False, 8, 2)
    _require_gfx950(q.device)
    _check_scale(sm_scale)
    if sm_scale is not None and torch.tensor(sm_scale, dtype=torch.float32).item() == 0:
        raise ValueError("sm_scale must be positive and finite FP32")
    with torch.cuda.device(q.device):
        if tensor_layout == "NHD":
            q, k, v = (x.transpose(1, 2) for x in (q, k, v))  # strided HND views, no copy
            B, H, N, D = q.shape
            out_nhd = torch.empty((B, N, H, D), dtype=q.dtype, device=q.device)
            out = out_nhd.transpose(1, 2)
        else:
            out_nhd = out = None
        result = forward_prepared(prepare(q, k, v, expcast=expcast, sm_scale=sm_scale), out=out)
        return out_nhd if out_nhd is not None else result


def fp8_kernel_resources(output_type=1, dim=128):
    """Compiled resources of the FP8 kernels (reference vc_fp8_kernel_resources,
    fp8_dispatch.cuh:61-73): {"fp8_control": {...}, "fp8_expcast": {...}}."""
    if output_type not in (0, 1) or dim not in (64, 128):
        raise ValueError("Expected output_type=0/1, D=64/128")
    ext = _extension()
    return {"fp8_control": ext.kernel_resources(dim, False, qk_fp8=True, expcast=False),
            "fp8_expcast": ext.kernel_resources(dim, False, qk_fp8=True, expcast=True)}
