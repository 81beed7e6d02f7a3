"""The C-ABI library: loads, exports every symbol of include/vcx.h, reports its
version and layout, and rejects invalid calls before any GPU work. CPU only:
no call here reaches a kernel launch."""
import ctypes
import re
from pathlib import Path

import pytest

import vcx

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "vcx.h").read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(vcx_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(vcx.LIB_PATH))
    names = declared_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(vcx.EXPORTED) == names


def test_abi_version_and_value_order():
    assert vcx.abi_version() == vcx.ABI_VERSION == 3
    tok = vcx.value_token()
    assert sorted(tok) == list(range(128))
    # closed form: position p = 32G + b holds token 16(b/4) + 8((b/2)%2) + 2G + b%2
    for p, t in enumerate(tok):
        G, b = divmod(p, 32)
        assert t == 16 * (b // 4) + 8 * ((b // 2) % 2) + 2 * G + b % 2
    # lane group G holds exactly the keys of Sage K-scale group (key % 8) // 2 == G
    for G in range(4):
        assert {(t % 8) // 2 for t in tok[32 * G:32 * G + 32]} == {G}
    assert vcx.lib().vcx_value_token(128) == -1


def test_workspace_sizes():
    for op in (vcx.WS_PREPARE_QK, vcx.WS_PREPARE_V, vcx.WS_GROUP):
        assert vcx.workspace_bytes(op, 1, 28, 37741, 128, True) > 0
    # grouping workspace grows with the cluster count and covers both schedules
    g = [vcx.workspace_bytes(vcx.WS_GROUP, 1, 28, 37741, 128, clusters=c) for c in (1, 8, 9, 64, 256)]
    assert g[2] < g[3] < g[4] and g[0] <= g[1]
    with pytest.raises(vcx.VcxError, match="clusters"):
        vcx.workspace_bytes(vcx.WS_GROUP, 1, 1, 100, 128, clusters=300)
    with pytest.raises(vcx.VcxError, match="unknown workspace op"):
        vcx.workspace_bytes(9, 1, 1, 1, 128)
    with pytest.raises(vcx.VcxError, match="invalid shape"):
        vcx.workspace_bytes(1, 1, 1, 1, 96)
    # the generic Q/K preprocessing takes any head dimension up to 128
    # fp64 tile sums [4 heads][1 tile][37] = 1184 B -> 1280, fp32 means 592 B -> 768 (256-byte aligned)
    assert vcx.workspace_bytes(vcx.WS_PREPROCESS_QK, 2, 2, 35, 37) == 1280 + 768
    with pytest.raises(vcx.VcxError, match="invalid shape"):
        vcx.workspace_bytes(vcx.WS_PREPROCESS_QK, 1, 1, 1, 129)


def _fwd(**kw):
    args = dict(q8=None, k8=None, v8=None, qs=None, ks=None, vs=None, means=None, B=1, H=1, Nq=1, Nk=1, D=128,
                expcast=1, block_values=0, channel_scale=1, sm=0.088, out_dtype=1, out=None, osb=128, osh=128,
                osn=128, pd=None, r0=0, r1=0, stream=None)
    args.update(kw)
    L = vcx.lib()
    rc = L.vcx_attention_fwd(*args.values())
    return rc, L.vcx_last_error().decode()


def test_invalid_calls_rejected_before_launch():
    assert _fwd(D=96) == (1, "D must be 64 or 128")
    rc, msg = _fwd(expcast=3)
    assert rc == 1 and "expcast" in msg
    rc, msg = _fwd(expcast=2, block_values=1)
    assert rc == 1 and "folded" in msg
    rc, msg = _fwd(expcast=0)  # the control path is accepted; the null pointers fail next
    assert rc == 1 and "null" in msg
    rc, msg = _fwd(sm=float("inf"))
    assert rc == 1 and "sm_scale" in msg
    rc, msg = _fwd()
    assert rc == 1 and "null" in msg
    rc, msg = _fwd(block_values=0, channel_scale=0)
    assert rc == 1 and "per-block" in msg
    L = vcx.lib()
    assert L.vcx_preprocess_qk(None, None, 2, 1, 1, 8, 8, 129, 0, 0, 129, 0, 0, 129, 1, 1, None, None, None, 0,
                               None) == 1
    assert "1..128" in L.vcx_last_error().decode()
    assert L.vcx_preprocess_qk(None, None, 3, 1, 1, 8, 8, 37, 0, 0, 37, 0, 0, 37, 1, 1, None, None, None, 0,
                               None) == 1
    assert "dtype" in L.vcx_last_error().decode()
    assert L.vcx_prepare_qk_int8_rotated(None, None, 1, 1, 1, 64, 128, 96, 0, 0, 96, 0, 0, 96, None,
                                         None, None, None, None, None, None, 0, None) == 1
    assert "D must be 64 or 128" in L.vcx_last_error().decode()
    assert L.vcx_prepare_qk_fp8(None, None, 1, 1, 1, 64, 128, 96, 0, 0, 96, 0, 0, 96,
                                None, None, None, None, None, None, 0, None) == 1
    assert "D must be 64 or 128" in L.vcx_last_error().decode()
    assert L.vcx_prepare_qk_fp8(None, None, 1, 1, 1, 64, 128, 128, 0, 0, 128, 0, 0, 128,
                                None, None, None, None, None, None, 0, None) == 1
    assert L.vcx_expcast_codes(None, None, -1, None) == 1
    # grouping: 1..256 clusters in either mode; anything else is rejected before a launch
    grp = lambda clusters, mode: L.vcx_group_values(None, 1, 1, 1, 10, 128, 0, 0, 128, clusters, 2, mode, None,
                                                    None, None, None, None, None, 0, None)
    assert grp(257, 0) == 1 and "[1, 256]" in L.vcx_last_error().decode()
    assert grp(16, 2) == 1 and "mode" in L.vcx_last_error().decode()
    assert grp(16, 1) == 1 and "v must be non-null" in L.vcx_last_error().decode()
    assert L.vcx_fp8_exp2_codes(None, None, 4, 0, None) == 1
    assert L.vcx_fp8_exp2_codes(ctypes.c_void_p(4096), ctypes.c_void_p(4096), 4, 2, None) == 1
    assert "form" in L.vcx_last_error().decode()
    # the allocation-free Q/K entry point refuses shapes beyond its 32 MiB scratch before any GPU call
    assert L.vcx_prepare_qk_int8_noalloc(None, None, 1, 1, 64, 128, 100000, 128, 0, 0, 128, 0, 0, 128, None,
                                         None, None, None, None, None, None) == 1
    assert "scratch" in L.vcx_last_error().decode()
    khz = ctypes.c_int(0)
    assert L.vcx_clock_probe(1000, None, ctypes.byref(khz), None) == 1
    assert "null" in L.vcx_last_error().decode()
    fake = ctypes.c_void_p(4096)  # never dereferenced: the window is checked first
    assert L.vcx_clock_probe(0, fake, ctypes.byref(khz), None) == 1
    assert "window_us" in L.vcx_last_error().decode()
    assert L.vcx_clock_probe(10000001, fake, ctypes.byref(khz), None) == 1
    assert L.vcx_clock_probe(1000, ctypes.c_void_p(4100), ctypes.byref(khz), None) == 1
    assert "aligned" in L.vcx_last_error().decode()


def test_python_binding_refuses_cpu_tensors():
    import torch
    with pytest.raises(vcx.VcxError, match="no CPU fallback"):
        vcx.prepare_qk(torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16), torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16))
