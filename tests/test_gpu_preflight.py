"""The hip backend's known-answer preflight (reference src/vc_attention/cuda_backend.py:97-129)
and the per-mode compiled-resource report under the reference's names, on the device."""
import pytest

pytestmark = pytest.mark.gpu


def test_preflight_passes_with_known_answers_and_build_info():
    print("case: preflight", flush=True)
    from vc_attention import preflight
    r = preflight("cuda:0")
    assert r["preflight"] == "passed" and r["arch"].startswith("gfx950")
    assert r["checks"]["expcast_known_answers"] == [120, 112, 107, 56, 8, 0, 0]
    assert r["abi_version"] >= 3 and r["default_kernel_mode"] == "optimized"


def test_kernel_resources_reference_names_on_device():
    print("case: kernel_resources", flush=True)
    from sageattention_local import kernel_resources
    for out_type in (0, 1):
        res = kernel_resources(out_type)
        for name in ("expcast_optimized", "expcast_vc15", "expcast_vc9", "smooth_optimized", "full_optimized",
                     "control_sage_layout_1", "expcast_sage_layout_35", "vc31_both"):
            row = res[name]
            assert 0 < row["registers_per_thread"] <= 256 and row["threads_per_block"] == 256, (name, row)
            assert row["predicted_active_blocks_per_sm"] >= 1, (name, row)
        # the main configuration's kernel (folded ExpCast, D128): two 128-row blocks per CU, no spills
        main = res["expcast_optimized"]
        assert main["predicted_active_blocks_per_sm"] == 2 and main["local_bytes_per_thread"] == 0, main
        # D64 with smoothing runs three blocks per CU (at most 168 registers)
        d64 = res["d64_full_optimized"]
        assert d64["predicted_active_blocks_per_sm"] == 3 and d64["registers_per_thread"] <= 168, d64
