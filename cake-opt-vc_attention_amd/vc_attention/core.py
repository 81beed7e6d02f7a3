"""``vc_attention`` surface with a ``hip`` backend for the sageattn_vc contract.

Mirrors the reference's src/vc_attention/core.py: a frozen ``Config`` with
validation (core.py:15-65), the request-scoped ``LayoutCache`` of the
denoising-step schedule with warm-started regrouping (core.py:153-226) and
``attention(...) -> (out, counters)`` with backend dispatch (core.py:263-371).

Backends of this build:
* ``"hip"``: the gfx950 sageattn_vc path (Sage per-thread INT8 QK, ExpCast or
  the Sage FP8 control probabilities (``expcast=False``), FP8 PV, optional V
  grouping + block smoothing) through libvcx. It requires ``qk_format="int8"``
  and the sageattn_vc block geometry (q_block=64, k_quant_block=128,
  kv_block=128, k_smooth=True, mean_dtype="float16", quantize=True).
  ``qk_hadamard=True`` rotates Q and the centred K by the normalized Sylvester
  transform (core.py:79-107's) inside the INT8 quantizers; ``False`` is the
  reference's sageattn_vc contract.
* ``"reference"``, ``"npu_fp8"``, ``"cuda_fp8"``: validated by ``Config``
  exactly as in the reference (core.py:36-65) so existing configurations keep
  constructing; ``attention`` raises NotImplementedError for them (the eager
  FP8-QK prototype and the Ascend/Hopper kernels are a different numerical
  contract that this build does not carry).
"""
import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Config:
    expcast: bool = False
    v_smooth: bool = False
    quantize: bool = True
    q_block: int = 128
    k_quant_block: int = 256
    kv_block: int = 128
    clusters: int = 8
    iterations: int = 2
    active_fraction: float = 0.25
    refresh_interval: int = 4
    mean_dtype: str = "float16"
    backend: str = "reference"
    k_smooth: bool = True
    qk_hadamard: bool = True
    cuda_schedule: str = "batched"
    cuda_fused_pipeline: bool = True
    cuda_fused_specialize: bool = True
    cuda_fused_interleave: bool = True
    qk_format: str = "fp8_block"

    def __post_init__(self):
        if self.cuda_schedule not in ("serial", "batched", "fused"):
            raise ValueError("cuda_schedule must be serial, batched, or fused")
        for name in ("expcast", "v_smooth", "quantize", "k_smooth", "qk_hadamard", "cuda_fused_pipeline",
                     "cuda_fused_specialize", "cuda_fused_interleave"):
            if not isinstance(getattr(self, name), bool):
                raise ValueError(f"{name} must be a bool")
        for name in ("q_block", "k_quant_block", "kv_block", "clusters", "iterations", "refresh_interval"):
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, int) or value < 1:
                raise ValueError(f"{name} must be a positive integer")
        if not math.isfinite(self.active_fraction) or not 0 <= self.active_fraction <= 1:
            raise ValueError("active_fraction must be in [0, 1]")
        if self.mean_dtype not in ("float16", "bfloat16", "float32"):
            raise ValueError("Unsupported mean_dtype")
        if self.backend not in ("reference", "npu_fp8", "cuda_fp8", "hip"):
            raise ValueError("backend must be reference, npu_fp8, cuda_fp8, or hip")
        if self.qk_format not in ("fp8_block", "int8"):
            raise ValueError("qk_format must be fp8_block or int8")
        if self.backend in ("npu_fp8", "cuda_fp8") and not self.quantize:
            raise ValueError(f"{self.backend} requires quantize=True")
        if self.backend in ("npu_fp8", "cuda_fp8") and self.k_quant_block % self.kv_block:
            raise ValueError(f"{self.backend} requires kv_block to divide k_quant_block")
        if self.backend == "cuda_fp8":
            if self.cuda_schedule == "fused" and self.kv_block != 128:
                raise ValueError("fused CUDA requires kv_block=128")
            if any(x < 32 or x > 256 or x % 32 for x in (self.q_block, self.kv_block)):
                raise ValueError("cuda_fp8 q_block/kv_block must be multiples of 32 in [32, 256]")
            if self.k_quant_block > 4096:
                raise ValueError("cuda_fp8 k_quant_block must be <= 4096")
        if self.backend == "hip":
            required = dict(qk_format="int8", quantize=True, q_block=64, k_quant_block=128,
                            kv_block=128, k_smooth=True, mean_dtype="float16")
            bad = [f"{k}={v!r}" for k, v in required.items() if getattr(self, k) != v]
            if bad:
                raise ValueError("hip backend implements the sageattn_vc contract; it requires " + ", ".join(bad))
            if self.clusters > 256:
                raise ValueError("hip backend groups V into at most 256 clusters")


@dataclass
class _LayerLayout:
    """What a layer keeps between denoising steps: the permutation and the grouping's next
    centers (the warm start of its next refresh), keyed by the V signature."""
    signature: tuple
    permutation: object
    centers: object
    refreshed_at: int
    last_step: int


class LayoutCache:
    """Request-scoped V layout of the denoising-step schedule (reference core.py:181-226).

    Within one request, a layer regroups V at the first step of its smoothing window and
    then every ``refresh_interval`` steps while smoothing is active (steps below
    ceil(total_steps * active_fraction)); between refreshes it reuses the permutation, while
    means and residuals are recomputed from the current V on every call. A refresh starts
    the grouping from the centers the previous refresh produced (the reference passes
    state["centers"] back, core.py:216-221). A new request id, a changed V shape / device /
    dtype / total_steps, or a step earlier than the layer's last one discards the layer's
    layout. ``layout`` returns (permutation or None, smoothing active, refreshed now).
    """

    def __init__(self, config):
        self.config = config
        self._request_id = None
        self._layers = {}

    @property
    def entries(self):
        return len(self._layers)

    def reset(self):
        self._request_id = None
        self._layers.clear()

    def _window(self, total_steps):
        """Number of leading steps with smoothing active."""
        return math.ceil(total_steps * self.config.active_fraction) if self.config.v_smooth else 0

    def _entry(self, layer_id, signature, step):
        """The layer's layout if it is still valid for this call, else None (and dropped)."""
        entry = self._layers.get(layer_id)
        if entry is not None and (entry.signature != signature or step < entry.last_step):
            del self._layers[layer_id]
            entry = None
        return entry

    def layout(self, v, *, step, total_steps, request_id, layer_id, grouping=None):
        if request_id is None:
            raise ValueError("A persistent layout cache requires request_id")
        if total_steps < 1 or not 0 <= step < total_steps:
            raise ValueError("Invalid denoising step/total_steps")
        if request_id != self._request_id:
            self.reset()
            self._request_id = request_id
        entry = self._entry(layer_id, (tuple(v.shape), str(v.device), v.dtype, total_steps), step)
        active = step < self._window(total_steps)
        due = active and (entry is None or step - entry.refreshed_at >= self.config.refresh_interval)
        if due:
            group = grouping if grouping is not None else _hip_grouping(self.config)
            perm, centers = group(v, None if entry is None else entry.centers)
            entry = _LayerLayout((tuple(v.shape), str(v.device), v.dtype, total_steps), perm, centers, step, step)
            self._layers[layer_id] = entry
        elif entry is not None:
            entry.last_step = step
        return (entry.permutation if entry is not None else None), active, due


def _hip_grouping(cfg):
    """grouping(v, centers or None) -> (permutation, next centers) on the GPU."""
    import vcx

    return lambda v, centers: vcx.group_values(v, cfg.clusters, cfg.iterations, centers=centers,
                                               return_centers=True)


def _validate(q, k, v, causal, mask):
    if causal:
        raise ValueError("This experiment does not support causal attention")
    if mask is not None:
        raise ValueError("This experiment does not support a mask/bias")
    if any(x.ndim != 4 for x in (q, k, v)):
        raise ValueError("Expected BNSD tensors")
    if q.shape[:2] != k.shape[:2] or k.shape[:2] != v.shape[:2]:
        raise ValueError("Batch and heads must match; GQA is not implemented")
    if k.shape[-2] != v.shape[-2] or q.shape[-1] != k.shape[-1] or v.shape[-1] != q.shape[-1]:
        raise ValueError("Incompatible Q/K/V shape")
    if any(0 in x.shape for x in (q, k, v)):
        raise ValueError("Empty Q/K/V are not supported")
    if any(x.device != q.device or x.dtype != q.dtype for x in (k, v)):
        raise ValueError("Q/K/V must have the same device and dtype")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("Inputs must be FP16/BF16/FP32 before quantization")
    if not all(bool(torch.isfinite(x).all()) for x in (q, k, v)):
        raise ValueError("Q/K/V must be finite")


@torch.no_grad()
def attention(q, k, v, config=None, *, cache=None, step=0, total_steps=1, request_id=None, layer_id=0,
              scale=None, causal=False, mask=None):
    """Return (output, counters) (reference core.py:263-371)."""
    cfg = config or Config()
    _validate(q, k, v, causal, mask)
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("scale must be positive and finite")
    if cfg.backend in ("npu_fp8", "cuda_fp8"):
        raise NotImplementedError(f"backend {cfg.backend!r} targets Ascend/Hopper kernels; on MI355X use "
                                  "Config(backend='hip', qk_format='int8', ...)")
    if cfg.backend != "hip":
        raise NotImplementedError("the eager FP8-QK reference backend is not part of this build; "
                                  "use Config(backend='hip', qk_format='int8', ...)")
    from sageattention_local import vc as sage

    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("hip backend requires FP16/BF16 inputs")
    if q.shape[-1] not in (64, 128):
        raise ValueError("hip backend requires head_dim 64 or 128")
    sage._require_gfx950(q.device)
    if cache is None:
        cache = LayoutCache(cfg)
        request_id = "one-shot" if request_id is None else request_id
    elif cache.config != cfg:
        raise ValueError("cache.config must match config")
    pi, active, refreshed = cache.layout(v, step=step, total_steps=total_steps, request_id=request_id,
                                         layer_id=layer_id)
    import vcx

    q8, qs, k8, ks, km = vcx.prepare_qk(q, k, pi, hadamard=cfg.qk_hadamard)
    v8, vs, means = vcx.prepare_v(v, pi, smooth=active, channel_scale=True)
    # The ExpCast encode of the reference's default kernel mode: folded without block values.
    out = vcx.forward(q8, k8, v8, qs, ks, vs, means, cfg.expcast, active, 0 if q.dtype == torch.float16 else 1,
                      scale, affine=cfg.expcast and not active)
    return out, {
        "backend": "hip",
        "smoothing_active": active,
        "layout_refreshed": refreshed,
        "expcast": cfg.expcast,
        "k_smooth": True,
        "qk_hadamard": cfg.qk_hadamard,
        "qk_format": "int8",
        "numerical_contract_version": "sageattn_vc-1",
        "tiles": math.ceil(q.shape[-2] / 128) * math.ceil(k.shape[-2] / 128),
        "native_fused_attention": True,
        "preprocessing_fused": True,
    }


def expcast_codes(shifted_scores):
    """ExpCast bytes of shifted scores via the gfx950 probe kernel (GPU tensors only)."""
    import vcx

    return vcx.expcast_codes(shifted_scores)
