"""Sage INT8 QK + VC V grouping/smoothing + ExpCast attention on MI355X (gfx950).

Drop-in for the reference's ``sageattention_local.vc`` module
(third_party/sageattention_local/sageattention_local/vc.py): same public
functions (``sageattn_vc``, ``prepare``, ``forward_prepared``,
``validate_inputs``, ``kernel_resources``, ``sage_vc_build_info``), same
argument meaning and the same ValueError checks before any native call. The
native work runs in libvcx.so (hand-written HIP for gfx950) through
:mod:`vcx`; there is no CPU fallback.

Differences a caller can observe, all deliberate:
* Any current HIP stream is accepted (the reference required the default
  stream because an upstream kernel used it); all work is enqueued on it.
* ``kernel_mode`` accepts the reference's documented mode names with the same
  compatibility rules. Every mode runs the single gfx950 kernel (the names
  select Hopper WGMMA/TMA schedules that have no MI355X counterpart); the
  numerics follow the mode as in the reference: without block values the
  default and vc12..vc15 modes use the folded ExpCast encode, vc4..vc11 the
  unfused one (``AFFINE_MODES``).
* The prepared ``v`` payload is stored in the gfx950 tile order
  (``vcx.value_token``), not Sage's 16-token permutation.
* ``expcast=False`` runs the Sage FP8 control path: each P byte is the E4M3 of
  the correctly rounded binary32 exp2 (hardware ``v_exp_f32``, rechecked in
  binary64 where an E4M3 rounding midpoint lies within two ulps), so the bytes
  are exact; the row mass sums the unrounded exp2 values.
"""
import math

import torch

import vcx

DEFAULT_EXPCAST_KERNEL = "vc15"
# Mode names of the reference (vc.py:14-46); values are the reference's schedule ids.
UNIFIED_MODES = {"vc31_unified": 38, "vc32_full_pv": 39, "vc32_packed_mean": 40}
DESCRIPTOR_CANDIDATES = {"vc30_desc": 37}
STREAM_CONVERT_CANDIDATES = {"vc28_stream_i2f": 35, "vc29_interleave_rows": 36}
PIPELINE_CANDIDATES = ("vc19_k", "vc19_v", "vc19_kv", "vc19_kv_late")
MASS_CANDIDATES = {"vc25_mass_serial": 7, "vc25_mass_overlap": 8}
DUAL_QUERY_CANDIDATES = {"vc26_shared": 1, "vc26_stagger": 2}
ENCODING_CANDIDATES = {"vc24_bitpack": 6}
STATE_CANDIDATES = {"vc23_maxstate": 4, "vc23_cached_bias": 5}
WORK_CANDIDATES = {"vc22_intmax": 1, "vc22_skip": 2, "vc22_both": 3}
HISTORY_CANDIDATES = {"vc21_history_r128": 128, "vc21_history_r168": 168}
COMPUTE_CANDIDATES = {"vc20_pv_qk": 1, "vc20_serial": 2, "vc20_qk_pv": 3}
SAGE_LAYOUT_MODES = {"vc16": 1, "vc16_early_v": 2, "vc16_pack_first": 3, "vc16_pack_early": 4, "vc16_serial": 5,
                     "vc17_g1": 6, "vc17_g4": 7, "vc17_c4": 8, "vc17_direct": 9,
                     "vc18_r128": 10, "vc18_r144": 11, "vc18_r192": 12,
                     "vc18_pv64_r128": 13, "vc18_pv64_r144": 14, "vc18_pv64_r168": 15,
                     **{mode: i + 16 for i, mode in enumerate(PIPELINE_CANDIDATES)},
                     **{mode: s + 19 for mode, s in COMPUTE_CANDIDATES.items()},
                     **{mode: i + 23 for i, mode in enumerate(HISTORY_CANDIDATES)},
                     **{mode: i + 24 for mode, i in WORK_CANDIDATES.items()},
                     **{mode: i + 24 for mode, i in STATE_CANDIDATES.items()},
                     **{mode: i + 24 for mode, i in ENCODING_CANDIDATES.items()},
                     **{mode: i + 24 for mode, i in MASS_CANDIDATES.items()},
                     **{mode: i + 32 for mode, i in DUAL_QUERY_CANDIDATES.items()},
                     **STREAM_CONVERT_CANDIDATES, **DESCRIPTOR_CANDIDATES, **UNIFIED_MODES}
BASE_MODES = ("optimized", "vc15", "vc14", "vc13_overlap", "vc13_serial", "vc12", "vc11", "vc10", "vc9",
              "vc7", "vc6", "vc4")


def _extension():
    """libvcx with its ABI checked (RuntimeError if missing or stale; never a fallback)."""
    vcx.lib()
    return vcx


def _check_mode(kernel_mode, *, v_smooth, expcast, dim, v_scale_mode):
    """Reference mode rules (vc.py:203-215 and :174-188)."""
    if kernel_mode not in BASE_MODES and kernel_mode not in SAGE_LAYOUT_MODES:
        raise ValueError("Unknown kernel_mode; use a documented vc4..vc21 mode or 'optimized'")
    if kernel_mode in UNIFIED_MODES and v_scale_mode != "channel":
        raise ValueError("vc31/vc32 require per-channel V scale")
    if kernel_mode in HISTORY_CANDIDATES and dim != 128:
        raise ValueError("Shared-history candidates require D128")
    if kernel_mode in SAGE_LAYOUT_MODES:
        schedule = SAGE_LAYOUT_MODES[kernel_mode]
        if v_smooth and kernel_mode not in UNIFIED_MODES:
            raise ValueError("Sage layout candidates require v_smooth=False")
        if 6 <= schedule <= 9 and not expcast:
            raise ValueError("Probability candidates require expcast=True")
        if expcast and schedule in (3, 4):
            raise ValueError("Pack-first candidates require expcast=False")


def validate_inputs(q, k, v, tensor_layout, is_causal, return_lse, expcast, v_smooth, clusters, iterations):
    """Same checks and messages as the reference (vc.py:121-138)."""
    if is_causal or return_lse:
        raise ValueError("Sage VC supports noncausal forward without LSE only")
    if tensor_layout not in ("HND", "NHD"):
        raise ValueError("tensor_layout must be HND or NHD")
    if not isinstance(expcast, bool) or not isinstance(v_smooth, bool):
        raise ValueError("expcast and v_smooth must be bool")
    if any(isinstance(x, bool) or not isinstance(x, int) for x in (clusters, iterations)) or \
            not (1 <= clusters <= 256 and 1 <= iterations <= 100):
        raise ValueError("Invalid clustering parameters")
    if any(x.ndim != 4 or x.numel() == 0 for x in (q, k, v)):
        raise ValueError("Expected nonempty four-dimensional Q/K/V")
    if q.dtype not in (torch.float16, torch.bfloat16) or any(x.dtype != q.dtype or x.device != q.device for x in (k, v)):
        raise ValueError("Q/K/V require matching FP16/BF16 dtype and device")
    head_axis = 1 if tensor_layout == "HND" else 2
    if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[head_axis] != k.shape[head_axis] \
            or q.shape[-1] != k.shape[-1]:
        raise ValueError("Q/K/V batch/heads/dim must match; GQA is unsupported")
    if q.shape[-1] not in (64, 128):
        raise ValueError("Sage VC requires D=64/128")


def _require_gfx950(device):
    if device.type != "cuda" or not torch.cuda.is_available():
        raise ValueError("Sage VC requires an MI355X (gfx950) GPU; no CPU/reference fallback")
    arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")
    if not arch.startswith("gfx950"):
        raise ValueError(f"Sage VC requires gfx950 (MI355X), found {arch or 'unknown'}; no fallback")


def _check_scale(sm_scale):
    if sm_scale is not None and (not math.isfinite(sm_scale) or not 0 < sm_scale <= 3.4028234663852886e38):
        raise ValueError("sm_scale must be positive and finite FP32")


@torch.no_grad()
def prepare(q, k, v, *, expcast=True, v_smooth=True, clusters=8, iterations=2, sm_scale=None,
            v_scale_mode="channel", grouping_mode="fused"):
    """HND preparation (reference vc.py:141-170) on the current stream.

    Grouping produces the permutation; K and V are gathered inside the
    quantizers (no permuted copies). ``v`` is in gfx950 tile storage order.
    grouping_mode="fused" is the reference's group_values (the fused schedule for at most
    8 effective clusters, the general one above); "legacy" runs the general schedule for
    every count, as group_values_legacy does (vc.py:153). Both follow one arithmetic
    contract, so they return the same permutation.
    """
    if v_scale_mode not in ("channel", "block"):
        raise ValueError("v_scale_mode must be 'channel' or 'block'")
    if grouping_mode not in ("fused", "legacy"):
        raise ValueError("grouping_mode must be 'fused' or 'legacy'")
    ext = _extension()
    permutation = ext.group_values(v, clusters, iterations, legacy=grouping_mode == "legacy") if v_smooth else None
    q8, qs, k8, ks, km = ext.prepare_qk(q, k, permutation)
    v8, vs, means = ext.prepare_v(v, permutation, smooth=v_smooth, channel_scale=v_scale_mode == "channel")
    return {"q": q8, "k": k8, "v": v8, "qs": qs, "ks": ks, "vs": vs, "means": means, "km": km,
            "expcast": expcast, "block_values": v_smooth, "output_type": 0 if q.dtype == torch.float16 else 1,
            "scale": q.shape[-1] ** -0.5 if sm_scale is None else sm_scale, "permutation": permutation,
            "v_layout": "gfx950_tile128"}


# Modes whose reference kernels fold RN(score*scale), the subtraction and the ExpCast map
# into one FMA (affine_probability, reference vc.py:187-189; FoldAffine, vc_sm90.cu:1009).
# The reference uses the folded encode only for ExpCast without block values.
AFFINE_MODES = ("optimized", "vc15", "vc14", "vc13_overlap", "vc13_serial", "vc12")


def forward_prepared(state, *, kernel_mode="optimized", out=None):
    """Fused kernel on a prepared state (reference vc.py:173-197)."""
    channel = not (state["block_values"] and state["vs"].ndim == 4)
    _check_mode(kernel_mode, v_smooth=state["block_values"] and kernel_mode not in UNIFIED_MODES,
                expcast=state["expcast"], dim=state["q"].shape[-1], v_scale_mode="channel" if channel else "block")
    if kernel_mode in UNIFIED_MODES and state["vs"].ndim != 3:
        raise ValueError("vc31/vc32 require per-channel V scale")
    mode = "vc15" if kernel_mode in SAGE_LAYOUT_MODES else kernel_mode
    affine = bool(state["expcast"]) and not state["block_values"] and mode in AFFINE_MODES
    return _extension().forward(state["q"], state["k"], state["v"], state["qs"], state["ks"], state["vs"],
                                state["means"], state["expcast"], state["block_values"], state["output_type"],
                                state["scale"], channel_scale=channel, affine=affine, out=out)


@torch.no_grad()
def sageattn_vc(q, k, v, tensor_layout="HND", is_causal=False, sm_scale=None, return_lse=False,
                *, expcast=True, v_smooth=True, clusters=8, iterations=2, kernel_mode="optimized",
                v_scale_mode="channel", grouping_mode="fused"):
    """Public entry (reference vc.py:200-235): noncausal, no LSE, D in {64,128}, fp16/bf16."""
    if kernel_mode not in BASE_MODES and kernel_mode not in SAGE_LAYOUT_MODES:
        raise ValueError("Unknown kernel_mode; use a documented vc4..vc21 mode or 'optimized'")
    if kernel_mode in UNIFIED_MODES and v_scale_mode != "channel":
        raise ValueError("vc31/vc32 require per-channel V scale")
    if kernel_mode in HISTORY_CANDIDATES and q.shape[-1] != 128:
        raise ValueError("Shared-history candidates require D128")
    if kernel_mode in SAGE_LAYOUT_MODES:
        _check_mode(kernel_mode, v_smooth=v_smooth, expcast=expcast, dim=q.shape[-1], v_scale_mode=v_scale_mode)
    if v_scale_mode not in ("channel", "block"):
        raise ValueError("v_scale_mode must be 'channel' or 'block'")
    if grouping_mode not in ("fused", "legacy"):
        raise ValueError("grouping_mode must be 'fused' or 'legacy'")
    validate_inputs(q, k, v, tensor_layout, is_causal, return_lse, expcast, v_smooth, clusters, iterations)
    _require_gfx950(q.device)
    _check_scale(sm_scale)
    with torch.cuda.device(q.device):
        if tensor_layout == "NHD":
            q, k, v = (x.transpose(1, 2) for x in (q, k, v))  # strided HND views, no copy
            B, H, N, D = q.shape
            out_nhd = torch.empty((B, N, H, D), dtype=q.dtype, device=q.device)
            out = out_nhd.transpose(1, 2)
        else:
            out_nhd = None
            out = None
        state = prepare(q, k, v, expcast=expcast, v_smooth=v_smooth, clusters=clusters, iterations=iterations,
                        sm_scale=sm_scale, v_scale_mode=v_scale_mode, grouping_mode=grouping_mode)
        result = forward_prepared(state, kernel_mode=kernel_mode, out=out)
        return out_nhd if out_nhd is not None else result


# The reference's kernel_resources names (vc_sm90.cu:801-808,1123-1213 and vc.py:113-118), each
# mapped to the (value mode, probability mode) of the gfx950 kernel this module launches for
# that mode at D128: value mode 0 = no block values, 1 = block values with channel scales;
# probability mode 0 = Sage FP8 control, 1 = unfused ExpCast, 2 = folded ExpCast
# (AFFINE_MODES without block values). "smooth_*" / "full_*" are the reference's
# block-value kernels without / with ExpCast; the sage-layout and vc31/vc32 entries follow
# forward_prepared's choice for those modes (sage-layout modes run as vc15).
_FOLDED, _UNFUSED, _CONTROL = (0, 2), (0, 1), (0, 0)
RESOURCE_MODES = {
    "smooth_vc7": (1, 0), "smooth_optimized": (1, 0), "full_vc7": (1, 1), "full_optimized": (1, 1),
    "expcast_vc9": _UNFUSED, "expcast_vc10": _UNFUSED, "expcast_vc11": _UNFUSED,
    "expcast_vc12": _FOLDED, "expcast_vc14": _FOLDED, "expcast_vc15": _FOLDED, "expcast_serial": _FOLDED,
    "expcast_optimized": _FOLDED, "expcast_vc13_overlap": _FOLDED,
    **{f"control_sage_layout_{n}": _CONTROL for n in (*range(1, 5), *range(10, 38))},
    **{f"expcast_sage_layout_{n}": _FOLDED for n in (1, 2, *range(5, 38))},
    "vc31_smooth": (1, 0), "vc31_both": (1, 1), "vc32_full_smooth": (1, 0), "vc32_full_both": (1, 1),
    "vc32_packed_smooth": (1, 0), "vc32_packed_both": (1, 1),
}
# Entries of this build without a reference name: the D64 kernels and the per-block-scale
# (v_scale_mode="block", value mode 2) kernels.
EXTRA_RESOURCE_MODES = {
    "d64_expcast_optimized": (64, 0, 2), "d64_expcast_vc9": (64, 0, 1), "d64_control": (64, 0, 0),
    "d64_full_optimized": (64, 1, 1), "d64_smooth_optimized": (64, 1, 0),
    "block_scale_full": (128, 2, 1), "block_scale_smooth": (128, 2, 0),
}


def kernel_resources(output_type=1):
    """Compiled resources per kernel mode under the reference's names (vc.py:113-118,
    vc_sm90.cu:786-822): registers_per_thread, local_bytes_per_thread (spill),
    static/dynamic_shared_bytes, threads_per_block, predicted_active_blocks_per_sm
    (per CU here). Each name reports the gfx950 kernel this module runs for that mode."""
    if output_type not in (0, 1) or isinstance(output_type, bool):
        raise RuntimeError("Output type must be 0 (FP16) or 1 (BF16)")
    ext = _extension()
    cache = {}

    def res(d, vm, pm):
        if (d, vm, pm) not in cache:
            cache[(d, vm, pm)] = ext.kernel_resources_mode(d, vm, pm, output_type)
        return dict(cache[(d, vm, pm)])

    out = {name: res(128, vm, pm) for name, (vm, pm) in RESOURCE_MODES.items()}
    out.update({name: res(d, vm, pm) for name, (d, vm, pm) in EXTRA_RESOURCE_MODES.items()})
    return out


def sage_vc_build_info():
    ext = _extension()
    return {"vc_extension": str(ext.LIB_PATH), "abi_version": ext.abi_version(), "arch": "gfx950",
            "algorithm": "Sage per-thread INT8 QK + VC block V residual/mean + ExpCast",
            "qk_hadamard": False, "v_block": 128, "mean_dtype": "float16",
            "clustering": "1..256 clusters, Lloyd with fp64 distances and tile-ordered fp64 center sums, stable "
                          "counting sort; fused schedule for <= 8 clusters, general schedule above or with "
                          "grouping_mode='legacy'; fresh every call",
            "expcast_probability": "without block values (default modes): folded encode RNE(fmaf(score, RN(scale*A), "
                                   "fmaf(-m, A, B))) with the 16-row |m| <= 128 fallback; otherwise exact FP32 RN "
                                   "multiply/subtract + single-rounding FMA + saturating RNE byte",
            "control_probability": "log2-domain FMA with the 8.807 offset; E4M3 (RNE) of the correctly rounded "
                                   "binary32 exp2 (v_exp_f32, binary64 recheck next to E4M3 midpoints); "
                                   "unrounded mass",
            "mass": "FP8 MFMA row sum with an all-ones operand (same accumulation as PV)",
            "v_layout": "gfx950_tile128", "kernel_modes": list(BASE_MODES) + list(SAGE_LAYOUT_MODES),
            "default_kernel_mode": "optimized"}
