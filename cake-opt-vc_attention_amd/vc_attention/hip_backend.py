"""Known-answer self-check of the hip backend before use.

Mirrors the reference's ``cuda_backend.preflight`` (src/vc_attention/cuda_backend.py:97-129):
fail loudly unless the native kernels give the published answers on this device, then
return the build's description. Checks, all on the GPU through libvcx:

* ExpCast bytes of the shifted scores [0, -1, -1.6, -8, -14, -100, -inf] / log2(e) equal
  the reference's known answers [120, 112, 107, 56, 8, 0, 0] (src tests test_core.py:17-22);
* attention of zero Q/K against constant V = 3 returns 3 on both probability paths
  (ExpCast and the Sage FP8 control), with and without V block smoothing, at a 19 x 35
  shape (partial tiles) and at 65 x 129 (two query blocks, a second key tile), D = 128:
  every logit is 0, so each row is the uniform average of V.
"""
import math

import torch

from .core import Config, attention, expcast_codes

EXPCAST_KA_INPUT = (0.0, -1.0, -1.6, -8.0, -14.0, -100.0, -math.inf)
EXPCAST_KA_CODES = (120, 112, 107, 56, 8, 0, 0)


def preflight(device="cuda:0"):
    """Run the known answers on `device`; RuntimeError if the device is not a gfx950 GPU,
    AssertionError if an answer is wrong. Returns a dict with "preflight": "passed"."""
    import vcx
    from sageattention_local import vc as sage

    device = torch.device(device)
    if device.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError("Preflight requires an MI355X (gfx950) GPU")
    arch = torch.cuda.get_device_properties(device).gcnArchName
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"Preflight requires an MI355X (gfx950) GPU, found {arch}")
    x = torch.tensor(EXPCAST_KA_INPUT, device=device) / math.log2(math.e)
    codes = expcast_codes(x).cpu().tolist()
    assert codes == list(EXPCAST_KA_CODES), f"ExpCast known answers: {codes}"
    shapes = ((19, 35), (65, 129))
    for nq, nk in shapes:
        q = torch.zeros(1, 1, nq, 128, device=device, dtype=torch.bfloat16)
        k = torch.zeros(1, 1, nk, 128, device=device, dtype=torch.bfloat16)
        v = torch.full((1, 1, nk, 128), 3.0, device=device, dtype=torch.bfloat16)
        for cast in (False, True):
            for smooth in (False, True):
                cfg = Config(backend="hip", qk_format="int8", q_block=64, k_quant_block=128, kv_block=128,
                             qk_hadamard=False, expcast=cast, v_smooth=smooth)
                actual, stats = attention(q, k, v, cfg)
                assert stats["backend"] == "hip" and stats["smoothing_active"] == smooth
                torch.testing.assert_close(actual.float(), torch.full_like(actual, 3).float(), rtol=2e-5, atol=2e-5)
    torch.cuda.synchronize(device)
    return {"device": str(device), "name": torch.cuda.get_device_name(device), "arch": arch,
            "preflight": "passed", "abi_version": vcx.abi_version(),
            "checks": {"expcast_known_answers": list(EXPCAST_KA_CODES),
                       "constant_v_attention": {"value": 3.0, "shapes": [list(s) for s in shapes],
                                                "expcast": [False, True], "v_smooth": [False, True]}},
            **sage.sage_vc_build_info()}
