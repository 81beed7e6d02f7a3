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
