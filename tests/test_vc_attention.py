"""CPU tests of the vc_attention surface: Config validation, the LayoutCache
denoising-step schedule and attention's argument checks.

Mirrors the reference's tests/test_core.py:96-143 (schedule, request reset,
unsupported semantics) and the Config rules of src/vc_attention/core.py:36-65.
The grouping callable is injected so the schedule runs without a GPU.
"""
import dataclasses

import pytest
import torch

from vc_attention import Config, LayoutCache, attention

HIP = dict(backend="hip", qk_format="int8", expcast=True, q_block=64, k_quant_block=128, kv_block=128,
           qk_hadamard=False)


def tensors(seed=3, nq=19, nk=35, heads=2, dim=16):
    gen = torch.Generator().manual_seed(seed)
    return [torch.randn(1, heads, n, dim, generator=gen) for n in (nq, nk, nk)]


def test_config_fields_and_defaults_match_reference():
    # src/vc_attention/core.py:15-34 (plus qk_format, this build's contract selector)
    got = {f.name: f.default for f in dataclasses.fields(Config)}
    ref = dict(expcast=False, v_smooth=False, quantize=True, q_block=128, k_quant_block=256, kv_block=128,
               clusters=8, iterations=2, active_fraction=0.25, refresh_interval=4, mean_dtype="float16",
               backend="reference", k_smooth=True, qk_hadamard=True, cuda_schedule="batched",
               cuda_fused_pipeline=True, cuda_fused_specialize=True, cuda_fused_interleave=True)
    for name, value in ref.items():
        assert got.pop(name) == value, name
    assert got == {"qk_format": "fp8_block"}


@pytest.mark.parametrize("kwargs, match", [
    (dict(cuda_schedule="eager"), "cuda_schedule"),
    (dict(k_smooth=1), "k_smooth must be a bool"),
    (dict(cuda_fused_pipeline=None), "cuda_fused_pipeline"),
    (dict(q_block=0), "q_block"),
    (dict(clusters=True), "clusters"),
    (dict(active_fraction=1.5), "active_fraction"),
    (dict(active_fraction=float("nan")), "active_fraction"),
    (dict(mean_dtype="float64"), "mean_dtype"),
    (dict(backend="triton"), "backend must be"),
    (dict(backend="cuda_fp8", quantize=False), "requires quantize=True"),
    (dict(backend="npu_fp8", k_quant_block=200), "divide k_quant_block"),
    (dict(backend="cuda_fp8", cuda_schedule="fused", kv_block=64, k_quant_block=256), "kv_block=128"),
    (dict(backend="cuda_fp8", q_block=48), "multiples of 32"),
    (dict(backend="cuda_fp8", k_quant_block=8192), "4096"),
    (dict(qk_format="int4"), "qk_format"),
    (dict(HIP, qk_format="fp8_block"), "qk_format='int8'"),
    (dict(HIP, q_block=128), "q_block=64"),
    (dict(HIP, mean_dtype="float32"), "mean_dtype='float16'"),
    (dict(HIP, clusters=257), "at most 256 clusters"),
])
def test_config_rejections(kwargs, match):
    with pytest.raises(ValueError, match=match):
        Config(**kwargs)


def test_config_accepts_reference_and_hip_configurations():
    Config()
    Config(backend="cuda_fp8", cuda_schedule="fused", q_block=64, kv_block=128, k_quant_block=256)
    Config(backend="npu_fp8", k_quant_block=256, kv_block=128)
    Config(**HIP, v_smooth=True, clusters=8, iterations=2)
    Config(**HIP, v_smooth=True, clusters=256, iterations=3)
    Config(**dict(HIP, expcast=False))  # the Sage FP8 control arm (reference replay.py:17)
    Config(**dict(HIP, qk_hadamard=True))  # Q/K rotation inside the INT8 quantizers


def _counting_grouping(calls):
    def grouping(v, centers):
        calls.append((tuple(v.shape), centers))
        return torch.argsort(v[..., 0], dim=-1, stable=True), ("centers", len(calls))
    return grouping


def test_cache_reuses_only_layout_and_resets_requests_and_shapes():
    # tests/test_core.py:96-115
    _, _, v = tensors()
    cfg = Config(**HIP, v_smooth=True, active_fraction=0.25, refresh_interval=4)
    cache = LayoutCache(cfg)
    calls = []
    g = _counting_grouping(calls)
    p0, active, refreshed = cache.layout(v, step=0, total_steps=20, request_id="a", layer_id=0, grouping=g)
    assert active and refreshed
    p1, active, refreshed = cache.layout(v + 1, step=1, total_steps=20, request_id="a", layer_id=0, grouping=g)
    assert active and not refreshed and p1 is p0
    _, active, refreshed = cache.layout(v, step=4, total_steps=20, request_id="a", layer_id=0, grouping=g)
    assert active and refreshed
    p5, active, refreshed = cache.layout(v, step=5, total_steps=20, request_id="a", layer_id=0, grouping=g)
    assert not active and not refreshed
    p6, _, _ = cache.layout(v, step=6, total_steps=20, request_id="a", layer_id=0, grouping=g)
    assert p6 is p5
    _, _, refreshed = cache.layout(v, step=0, total_steps=20, request_id="b", layer_id=0, grouping=g)
    assert refreshed and cache.entries == 1
    _, _, refreshed = cache.layout(v[:, :, :-1], step=1, total_steps=20, request_id="b", layer_id=0, grouping=g)
    assert refreshed
    assert len(calls) == 4


def test_cache_refresh_warm_starts_from_the_previous_centers():
    # src/vc_attention/core.py:216-221: a refresh passes the cached centers to the grouping;
    # the first grouping of a layer (and any after a reset) starts cold.
    _, _, v = tensors()
    cache = LayoutCache(Config(**HIP, v_smooth=True, active_fraction=1.0, refresh_interval=2))
    calls = []
    g = _counting_grouping(calls)
    for step in range(6):
        cache.layout(v, step=step, total_steps=6, request_id="r", layer_id=7, grouping=g)
    assert [c for _, c in calls] == [None, ("centers", 1), ("centers", 2)]
    cache.layout(v, step=0, total_steps=6, request_id="next", layer_id=7, grouping=g)
    assert calls[-1][1] is None
    cache.layout(v[:, :1], step=2, total_steps=6, request_id="next", layer_id=7, grouping=g)
    assert calls[-1][1] is None and len(calls) == 5  # a new V shape is a new layout


def test_cache_layers_are_independent_and_step_regression_resets():
    _, _, v = tensors()
    cache = LayoutCache(Config(**HIP, v_smooth=True, active_fraction=1.0, refresh_interval=3))
    calls = []
    g = _counting_grouping(calls)
    a, _, _ = cache.layout(v, step=0, total_steps=10, request_id="r", layer_id=0, grouping=g)
    b, _, _ = cache.layout(v, step=0, total_steps=10, request_id="r", layer_id=1, grouping=g)
    assert cache.entries == 2 and a is not b
    _, _, refreshed = cache.layout(v, step=2, total_steps=10, request_id="r", layer_id=0, grouping=g)
    assert not refreshed
    _, _, refreshed = cache.layout(v, step=1, total_steps=10, request_id="r", layer_id=0, grouping=g)
    assert refreshed  # a step earlier than the cached one starts over


def test_cache_without_smoothing_never_groups():
    _, _, v = tensors()
    cache = LayoutCache(Config(**HIP, v_smooth=False))
    calls = []
    pi, active, refreshed = cache.layout(v, step=0, total_steps=4, request_id="a", layer_id=0,
                                         grouping=_counting_grouping(calls))
    assert pi is None and not active and not refreshed and not calls


@pytest.mark.parametrize("kwargs, match", [
    (dict(request_id=None), "request_id"),
    (dict(step=4), "step"),
    (dict(total_steps=0, step=0), "step"),
])
def test_cache_argument_errors(kwargs, match):
    _, _, v = tensors()
    args = dict(step=0, total_steps=4, request_id="a", layer_id=0)
    args.update(kwargs)
    with pytest.raises(ValueError, match=match):
        LayoutCache(Config(**HIP, v_smooth=True)).layout(v, **args)


def test_unsupported_semantics_fail_explicitly():
    # tests/test_core.py:127-137
    q, k, v = tensors()
    cfg = Config(**HIP)
    with pytest.raises(ValueError, match="causal"):
        attention(q, k, v, cfg, causal=True)
    with pytest.raises(ValueError, match="mask"):
        attention(q, k, v, cfg, mask=torch.ones(19, 35))
    with pytest.raises(ValueError, match="heads"):
        attention(q, k[:, :1], v[:, :1], cfg)
    with pytest.raises(ValueError, match="finite"):
        attention(q * float("nan"), k, v, cfg)


def test_other_backends_and_cpu_tensors_have_no_fallback():
    q, k, v = tensors(dim=64)
    for cfg in (Config(), Config(backend="cuda_fp8"), Config(backend="npu_fp8")):
        with pytest.raises(NotImplementedError):
            attention(q, k, v, cfg)
    with pytest.raises(ValueError, match="FP16/BF16"):
        attention(q, k, v, Config(**HIP))
    with pytest.raises(ValueError, match="gfx950"):
        attention(*(x.to(torch.bfloat16) for x in (q, k, v)), Config(**HIP))


def test_preflight_requires_a_gfx950_device():
    # reference cuda_backend.py:101-102: the preflight refuses anything but its GPU class
    from vc_attention import preflight
    with pytest.raises(RuntimeError, match="gfx950"):
        preflight("cpu")
