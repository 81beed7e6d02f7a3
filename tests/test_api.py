"""The Python surface (sageattention_local.vc): the reference's argument checks,
raised before any native call, and dispatch of prepared states to libvcx.
Mirrors the reference's tests/test_sage_vc.py:108-207 for this build. CPU only."""
from types import SimpleNamespace

import pytest
import torch

from sageattention_local import vc as api


@pytest.mark.parametrize("kwargs,match", [
    ({"is_causal": True}, "noncausal"), ({"return_lse": True}, "LSE"),
    ({"tensor_layout": "XYZ"}, "tensor_layout"), ({"expcast": 1}, "bool"),
    ({"clusters": 0}, "clustering"), ({"iterations": True}, "clustering"),
    ({"kernel_mode": "unknown"}, "kernel_mode"),
    ({"v_scale_mode": "unknown"}, "v_scale_mode"),
])
def test_unsupported_modes_rejected_before_native_dispatch(kwargs, match):
    q = torch.zeros(1, 2, 5, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match=match):
        api.sageattn_vc(q, q, q, **kwargs)


def test_gqa_cpu_and_mixed_dtypes_are_not_silent_fallbacks():
    q = torch.zeros(1, 2, 5, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="GQA"):
        api.sageattn_vc(q, q[:, :1], q[:, :1])
    with pytest.raises(ValueError, match="matching"):
        api.sageattn_vc(q, q.float(), q)
    with pytest.raises(ValueError, match="gfx950"):
        api.sageattn_vc(q, q, q)


@pytest.mark.parametrize("mode", list(api.SAGE_LAYOUT_MODES))
def test_sage_layout_mode_rules_match_reference(mode):
    schedule = api.SAGE_LAYOUT_MODES[mode]
    dim = 128 if mode in api.HISTORY_CANDIDATES else 64
    q = torch.zeros(1, 2, 5, dim, dtype=torch.float16)
    if mode not in api.UNIFIED_MODES:
        with pytest.raises(ValueError, match="v_smooth=False"):
            api.sageattn_vc(q, q, q, kernel_mode=mode)
    if schedule in (3, 4):
        with pytest.raises(ValueError, match="expcast=False"):
            api.sageattn_vc(q, q, q, kernel_mode=mode, v_smooth=False)


@pytest.mark.parametrize("mode", list(api.HISTORY_CANDIDATES))
def test_shared_history_rejects_d64_before_native_dispatch(monkeypatch, mode):
    def forbidden():
        raise AssertionError("Native extension must not load")
    monkeypatch.setattr(api, "_extension", forbidden)
    q = torch.zeros(1, 1, 65, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="D128"):
        api.sageattn_vc(q, q, q, v_smooth=False, kernel_mode=mode)


def payload(block_values, vs_ndim=3):
    return {"q": torch.zeros(1, 1, 65, 64, dtype=torch.int8), "k": torch.zeros(1, 1, 129, 64, dtype=torch.int8),
            "v": torch.zeros(1, 1, 64, 256, dtype=torch.uint8), "qs": torch.ones(1, 1, 64), "ks": torch.ones(1, 1, 8),
            "vs": torch.ones(1, 1, 64) if vs_ndim == 3 else torch.ones(1, 1, 2, 64),
            "means": torch.zeros(1, 1, 2, 64, dtype=torch.float16), "expcast": True, "block_values": block_values,
            "output_type": 1, "scale": 0.125}


@pytest.mark.parametrize("mode", ["optimized", "vc15", "vc4", "vc22_both", "vc28_stream_i2f"])
def test_forward_prepared_dispatches_state_to_the_single_kernel(monkeypatch, mode):
    calls = []
    monkeypatch.setattr(api, "_extension", lambda: SimpleNamespace(forward=lambda *a, **k: calls.append((a, k)) or "out"))
    state = payload(False)
    assert api.forward_prepared(state, kernel_mode=mode) == "out"
    (args, kwargs), = calls
    assert args[:7] == tuple(state[x] for x in ("q", "k", "v", "qs", "ks", "vs", "means"))
    assert args[7:] == (True, False, 1, 0.125)
    assert kwargs["channel_scale"] is True
    # reference vc.py:187-189: the default and vc12..vc15 modes fold the ExpCast encode
    assert kwargs["affine"] is (mode in ("optimized", "vc15", "vc22_both", "vc28_stream_i2f"))


def test_folded_encode_never_with_block_values_or_control(monkeypatch):
    calls = []
    monkeypatch.setattr(api, "_extension", lambda: SimpleNamespace(forward=lambda *a, **k: calls.append(k) or "out"))
    api.forward_prepared(payload(True))
    api.forward_prepared({**payload(False), "expcast": False})
    api.forward_prepared(payload(False), kernel_mode="vc11")
    assert [k["affine"] for k in calls] == [False, False, False]


def test_forward_prepared_block_scales_dispatch_without_channel_scale(monkeypatch):
    # reference vc.py:161, 180-190: per-block V scales ([B,H,tiles,D]) reach the kernel as block values
    calls = []
    monkeypatch.setattr(api, "_extension", lambda: SimpleNamespace(forward=lambda *a, **k: calls.append((a, k)) or "out"))
    assert api.forward_prepared(payload(True, vs_ndim=4)) == "out"
    (args, kwargs), = calls
    assert args[7:9] == (True, True) and kwargs["channel_scale"] is False


def test_forward_prepared_control_path_dispatches_expcast_false(monkeypatch):
    # reference vc.py:173-197: expcast=False selects the Sage FP8 control probabilities
    calls = []
    monkeypatch.setattr(api, "_extension", lambda: SimpleNamespace(forward=lambda *a, **k: calls.append((a, k)) or "out"))
    assert api.forward_prepared({**payload(False), "expcast": False}) == "out"
    (args, _), = calls
    assert args[7] is False


def test_forward_prepared_rejections(monkeypatch):
    monkeypatch.setattr(api, "_extension", lambda: SimpleNamespace(forward=lambda *a, **k: "out"))
    with pytest.raises(ValueError, match="per-channel V scale"):
        api.forward_prepared(payload(True, vs_ndim=4), kernel_mode="vc31_unified")
    with pytest.raises(ValueError, match="v_smooth=False"):
        api.forward_prepared(payload(True), kernel_mode="vc16")


# ---- binding-level checks (vcx): raised before the library is touched, so no kernel runs

import vcx  # noqa: E402


@pytest.fixture
def no_native(monkeypatch):
    def forbidden():
        raise AssertionError("libvcx must not be called")
    monkeypatch.setattr(vcx, "lib", forbidden)


@pytest.mark.parametrize("bad", ["short", "dtype", "wide"])
def test_forward_rejects_a_mismatched_out_buffer(no_native, bad):
    st = payload(False)
    B, H, Nq, D = st["q"].shape
    out = {"short": torch.empty(B, H, Nq - 1, D, dtype=torch.bfloat16),
           "dtype": torch.empty(B, H, Nq, D, dtype=torch.uint8),
           "wide": torch.empty(B, H, Nq, D, dtype=torch.float32)}[bad]
    with pytest.raises(vcx.VcxError, match="out must be"):
        vcx.forward(*(st[x] for x in ("q", "k", "v", "qs", "ks", "vs", "means")), True, False, 1, 0.125, out=out)


def test_forward_fp8_rejects_a_mismatched_out_buffer(no_native):
    q8 = torch.zeros(1, 1, 65, 64, dtype=torch.uint8)
    k8 = torch.zeros(1, 1, 129, 64, dtype=torch.uint8)
    v8 = torch.zeros(1, 1, 64, 256, dtype=torch.uint8)
    qs, ks, vs = torch.ones(1, 1, 2), torch.ones(1, 1, 2), torch.ones(1, 1, 64)
    with pytest.raises(vcx.VcxError, match="out must be"):
        vcx.forward_fp8(q8, k8, v8, qs, ks, vs, True, 1, 0.125, out=torch.empty(1, 1, 64, 64, dtype=torch.bfloat16))
    with pytest.raises(vcx.VcxError, match="out must be"):
        vcx.forward_fp8(q8, k8, v8, qs, ks, vs, True, 0, 0.125, out=torch.empty(1, 1, 65, 64, dtype=torch.bfloat16))


@pytest.mark.parametrize("kshape", [(1, 1, 40, 128), (2, 2, 40, 128), (1, 2, 40, 64)])
@pytest.mark.parametrize("fn", ["prepare_qk", "prepare_qk_fp8"])
def test_prepare_qk_rejects_k_that_does_not_match_q(no_native, fn, kshape):
    q = torch.zeros(1, 2, 33, 128, dtype=torch.bfloat16)
    k = torch.zeros(*kshape, dtype=torch.bfloat16)
    with pytest.raises(vcx.VcxError, match="must match in batch, heads and head dim"):
        getattr(vcx, fn)(q, k)


def test_kernel_resources_answer_under_the_reference_names(monkeypatch):
    # reference vc.py:113-118 and vc_sm90.cu:801-808,1123-1213: callers read
    # resources["expcast_optimized"], ["smooth_optimized"], ["expcast_sage_layout_35"], ...
    calls = []

    def fake(d, vm, pm, out_type):
        calls.append((d, vm, pm, out_type))
        return {"registers_per_thread": 100 * vm + 10 * pm + d // 64, "local_bytes_per_thread": 0,
                "static_shared_bytes": 0, "dynamic_shared_bytes": 0, "threads_per_block": 256,
                "predicted_active_blocks_per_sm": 2}

    monkeypatch.setattr(api, "_extension", lambda: SimpleNamespace(kernel_resources_mode=fake))
    res = api.kernel_resources(0)
    reg = lambda name: res[name]["registers_per_thread"]
    # folded ExpCast without block values: the default and vc12..vc15 modes, and the
    # sage-layout modes (which run as vc15)
    for name in ("expcast_optimized", "expcast_vc15", "expcast_vc14", "expcast_vc12", "expcast_vc13_overlap",
                 "expcast_serial", "expcast_sage_layout_35", "expcast_sage_layout_1"):
        assert reg(name) == 22, name
    for name in ("expcast_vc9", "expcast_vc10", "expcast_vc11"):  # unfused ExpCast
        assert reg(name) == 12, name
    for name in ("control_sage_layout_1", "control_sage_layout_37"):  # control path
        assert reg(name) == 2, name
    # block values: "smooth" without ExpCast, "full" and vc31/vc32 "both" with it
    for name in ("smooth_vc7", "smooth_optimized", "vc31_smooth", "vc32_full_smooth", "vc32_packed_smooth"):
        assert reg(name) == 102, name
    for name in ("full_vc7", "full_optimized", "vc31_both", "vc32_full_both", "vc32_packed_both"):
        assert reg(name) == 112, name
    assert reg("d64_expcast_optimized") == 21 and reg("block_scale_full") == 212
    assert {c[3] for c in calls} == {0} and {c[0] for c in calls} == {64, 128}
    assert len(calls) == len(set(calls))  # each kernel queried once
    assert set(res["expcast_optimized"]) == {"registers_per_thread", "local_bytes_per_thread", "static_shared_bytes",
                                             "dynamic_shared_bytes", "threads_per_block",
                                             "predicted_active_blocks_per_sm"}
    for bad in (2, -1, True):
        with pytest.raises(RuntimeError, match="Output type"):
            api.kernel_resources(bad)
