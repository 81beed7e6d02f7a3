"""GPU parity of the block-scaled FP8 QK path (the reference's experimental vc27)
through libvcx's C ABI against the CPU oracle.

Bit-exact: K channel mean (binary32), Q/K E4M3 codes and block scales. The cases
follow the reference's vc27 quantization gate (scripts/validate_fp8_qk.py:23-55):
fp16/bf16, D 64/128, ragged Nq/Nk around the 64/128-row blocks, per-channel K
offsets, a 3x Q block, constant inputs 0/8/10000 (whose centred K is exactly zero,
giving zero codes and the 1e-12 scale floor), plus strided NHD input.
"""
import numpy as np
import pytest
import torch

import vcx
from helpers import bits, dtype_name
from oracle import vc_oracle as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

GATE_SIZES = [(1, 1), (63, 127), (64, 128), (65, 129), (193, 513), (129, 4097)]


def _print_case(*args):
    print("case:", *args, flush=True)


def _gate_inputs(nq, nk, D, dt, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(2, 3, nq, D, generator=g).to(dt)
    k = torch.randn(2, 3, nk, D, generator=g).to(dt)
    k += (torch.arange(D, dtype=torch.float32) / 4).to(dt).view(1, 1, 1, -1)
    q[:, :, 64:] *= 3
    return q, k


def _check_prepare(q, k, qd=None, kd=None):
    name = dtype_name(q.dtype)
    q8, qs, k8, ks, km = vcx.prepare_qk_fp8(q.to(DEV) if qd is None else qd, k.to(DEV) if kd is None else kd)
    ekm = o.k_mean_f32(bits(k), name)
    eq8, eqs = o.quant_fp8_block(bits(q), 64, None, name)
    ek8, eks = o.quant_fp8_block(bits(k), 128, ekm, name)
    np.testing.assert_array_equal(km.cpu().numpy().view(np.uint32), ekm.view(np.uint32))
    np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint32), eqs.view(np.uint32))
    np.testing.assert_array_equal(q8.cpu().numpy(), eq8)
    np.testing.assert_array_equal(ks.cpu().numpy().view(np.uint32), eks.view(np.uint32))
    np.testing.assert_array_equal(k8.cpu().numpy(), ek8)
    return q8, qs, k8, ks, km


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("nq,nk", GATE_SIZES)
def test_prepare_qk_fp8_bit_exact(nq, nk, D, dt):
    _print_case("prepare_qk_fp8", nq, nk, D, dt)
    q, k = _gate_inputs(nq, nk, D, dt, seed=2701 + nq + nk + D)
    _check_prepare(q, k)


@pytest.mark.parametrize("value", [0.0, 8.0, 10000.0])
@pytest.mark.parametrize("D", [64, 128])
def test_prepare_qk_fp8_constant_inputs(value, D):
    _print_case("prepare_qk_fp8 constant", value, D)
    q = torch.full((1, 2, 65, D), value, dtype=torch.bfloat16)
    k = torch.full((1, 2, 129, D), value, dtype=torch.bfloat16)
    q8, qs, k8, ks, km = _check_prepare(q, k)
    assert torch.all(km.cpu() == k[0, 0, 0, 0].float())
    assert int(torch.count_nonzero(k8)) == 0
    assert torch.all(ks.cpu() == torch.tensor(1e-12, dtype=torch.float32))
    assert torch.isfinite(qs).all()


def test_prepare_qk_fp8_strided_nhd():
    B, H, N, D = 1, 3, 333, 128
    q, k = _gate_inputs(N, N, D, torch.bfloat16, seed=11)
    q, k = q[:B], k[:B]
    qn, kn = (x.transpose(1, 2).contiguous().to(DEV) for x in (q, k))
    _print_case("prepare_qk_fp8 NHD", B, H, N, D)
    _check_prepare(q, k, qn.transpose(1, 2), kn.transpose(1, 2))


# ------------------------------------------------------------------ fused FP8 forward

from helpers import cosine, logical_to_storage, make_qkv, output_bound, storage_to_logical  # noqa: E402

MODES = {"folded": (True, True), "unfused": (True, False), "control": (False, False)}  # expcast, affine


def _to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _run(st, expcast, affine, rows):
    tok = vcx.value_token()
    v8 = _to_dev(logical_to_storage(st["v"], tok))
    return vcx.forward_fp8(_to_dev(st["q"]), _to_dev(st["k"]), v8, _to_dev(st["qs"]), _to_dev(st["ks"]),
                           _to_dev(st["vs"]), expcast, st["output_type"], st["scale"], affine=affine, p_rows=rows)


def _integer_state(B, H, Nq, Nk, D, seed, dtype="bfloat16"):
    """FP8 payloads whose Q/K codes are integers in [-8, 8]: every E4M3 product is an
    integer of magnitude <= 64 and every score an integer below 2^13, so the FP8 MFMA's
    score equals the exact sum and the P bytes are fixed exactly."""
    rng = np.random.default_rng(seed)
    tiles = (Nk + 127) // 128
    q = o.e4m3_encode(rng.integers(-8, 9, (B, H, Nq, D)).astype(np.float32))
    k = o.e4m3_encode(rng.integers(-8, 9, (B, H, Nk, D)).astype(np.float32))
    # scales in [1/8, 1/2): logits of standard deviation about 0.4 to 6
    qs = np.ldexp(rng.uniform(1, 2, (B, H, (Nq + 63) // 64)), rng.integers(-3, -1, (B, H, (Nq + 63) // 64)))
    ks = np.ldexp(rng.uniform(1, 2, (B, H, tiles)), rng.integers(-3, -1, (B, H, tiles)))
    v = rng.integers(0, 256, (B, H, D, tiles * 128)).astype(np.uint8)
    v[(v & 0x7F) == 0x7F] = 0  # no NaN codes
    v[..., Nk:] = 0
    vs = rng.uniform(0.001, 0.01, (B, H, D)).astype(np.float32)
    return {"q": q, "k": k, "v": v, "qs": qs.astype(np.float32), "ks": ks.astype(np.float32), "vs": vs,
            "means": None, "qk_format": "fp8_block", "block_values": False,
            "output_type": 1 if dtype == "bfloat16" else 0, "scale": D ** -0.5}


INT_CASES = [  # B, H, Nq, Nk, D
    (1, 2, 256, 1024, 128),
    (2, 3, 65, 129, 64),
    (1, 1, 1, 1, 128),
    (1, 2, 200, 385, 128),
    (1, 1, 63, 4097, 64),
]


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("case", INT_CASES, ids=lambda c: "B%dH%dq%dk%dD%d" % c)
def test_fp8_forward_exact_scores_p_bytes_bit_exact(case, mode):
    B, H, Nq, Nk, D = case
    expcast, affine = MODES[mode]
    _print_case("fp8 forward integer codes", case, mode)
    st = _integer_state(B, H, Nq, Nk, D, seed=Nq * 7 + Nk)
    st["expcast"] = expcast
    out, pd = _run(st, expcast, affine, (0, Nq))
    eout, ecodes = o.reference(st, return_codes=True, affine=affine)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out.float().cpu().numpy()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound), float((err - bound).max())
    assert cosine(got, eout) >= 0.9999


FWD_CASES = [  # B, H, Nq, Nk, D, dtype
    (1, 2, 2048, 2048, 128, torch.bfloat16),
    (2, 3, 65, 129, 64, torch.float16),
    (1, 2, 257, 385, 128, torch.float16),
    (1, 1, 200, 4097, 128, torch.bfloat16),
]


def _expected_from_codes(st, codes, expcast):
    """The output implied by given P bytes: per row, sum_t w_t * sum_k dec(code) * V over
    sum_t w_t * mass_t, times the channel V scale, where w_t rescales tile t from its
    running maximum m_t to the final one (ExpCast: exp(m_t - m_T), masses are the decoded
    bytes; control: exp2(m_t - m_T), masses are the unrounded exp2 values). Logits in
    float64 from the decoded payloads: their rounding moves m_t by ulps, far below the
    output tolerance."""
    dec = o.e4m3_decode
    q, k = dec(st["q"]).astype(np.float64), dec(st["k"]).astype(np.float64)
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    tiles = (Nk + 127) // 128
    vdec = dec(st["v"]).astype(np.float64)  # [B,H,D,tiles*128] logical
    sm = float(np.float32(st["scale"])) * (1.0 if expcast else 1.4426950408889634)
    qs = np.repeat(st["qs"].astype(np.float64), 64, axis=2)[:, :, :Nq]
    ks = np.repeat(st["ks"].astype(np.float64), 128, axis=2)[:, :, :Nk]
    logit = (q @ np.swapaxes(k, 2, 3)) * qs[..., None] * ks[:, :, None, :] * sm
    pad = np.full((B, H, Nq, tiles * 128 - Nk), -np.inf)
    logit = np.concatenate([logit, pad], axis=3).reshape(B, H, Nq, tiles, 128)
    tmax = logit.max(axis=4) - (0.0 if expcast else 8.807)
    m = np.maximum.accumulate(np.maximum(tmax, -5e6), axis=3)  # running max after tile t
    p = dec(codes).astype(np.float64).reshape(B, H, Nq, tiles, 128)
    if expcast:
        w = np.exp(m - m[..., -1:])
        mass = p.sum(axis=4)
    else:
        w = np.exp2(m - m[..., -1:])
        mass = np.exp2(logit - m[..., None]).sum(axis=4)
    num = (p * w[..., None]).reshape(B, H, Nq, tiles * 128) @ np.swapaxes(vdec, 2, 3)
    den = (w * mass).sum(axis=3)
    return num / den[..., None] * st["vs"].astype(np.float64)[:, :, None, :]


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("case", FWD_CASES, ids=lambda c: "B%dH%dq%dk%dD%d" % c[:5])
def test_fp8_forward_gaussian_p_bytes_and_output(case, mode):
    """Quantized N(0,1) inputs. The FP8 MFMA accumulates the 128 E4M3 products with a
    finite alignment window, so a score can differ from the exactly rounded sum in its
    last bits; a P byte may then move by one code. Bound: at most 1 in 2000 bytes differ,
    none by more than one code; the output within the bf16/fp16 bound of the attention
    its own P bytes define, and cosine >= 0.9999 against the oracle's output."""
    B, H, Nq, Nk, D, dt = case
    expcast, affine = MODES[mode]
    _print_case("fp8 forward gaussian", case, mode)
    q, k, v = make_qkv(B, H, Nq, Nk, D, dt, seed=27)
    st = o.prepare_fp8(bits(q), bits(k), bits(v), expcast=expcast, dtype=dtype_name(dt))
    out, pd = _run(st, expcast, affine, (0, Nq))
    eout, ecodes = o.reference(st, return_codes=True, affine=affine)
    got_codes = pd.cpu().numpy()
    # ExpCast codes, and E4M3 codes of nonnegative probabilities, are monotone in the byte
    diff = np.abs(got_codes.astype(np.int32) - ecodes.astype(np.int32))
    frac = float((diff != 0).mean())
    print("P byte mismatches:", int((diff != 0).sum()), "of", diff.size, "max", int(diff.max()), flush=True)
    assert diff.max() <= 1
    assert frac <= 5e-4
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    # the kernel's output is the attention its own P bytes define ...
    err, bound = output_bound(got, _expected_from_codes(st, got_codes, expcast))
    assert np.all(err <= bound), float((err - bound).max())
    # ... and the rare one-code moves leave it next to the oracle's
    assert cosine(got, eout) >= 0.9999


@pytest.mark.parametrize("cast", [False, True])
@pytest.mark.parametrize("nk", [1, 129, 257])
def test_fp8_zero_logits_tail_and_v_scale_known_answer(cast, nk):
    # tests/test_fp8_qk.py:45-57: Q = K = 0, V = 2 on the valid keys, vs = 3.
    # ExpCast: every weight is 1, out = 6. Control: P = E4M3(2^8.807) = 448 over an
    # unrounded mass 2^8.807 per key, out = 6 * 448 / 2^8.807.
    D, nq = 64, 65
    tiles = (nk + 127) // 128
    v = np.zeros((1, 1, D, tiles * 128), np.uint8)
    v[..., :nk] = o.e4m3_encode(np.float32(2.0))
    st = {"q": np.zeros((1, 1, nq, D), np.uint8), "k": np.zeros((1, 1, nk, D), np.uint8), "v": v,
          "qs": np.ones((1, 1, 2), np.float32), "ks": np.ones((1, 1, tiles), np.float32),
          "vs": np.full((1, 1, D), 3.0, np.float32), "output_type": 1, "scale": 0.125}
    out = _run(st, cast, cast, None).float().cpu().numpy()
    weight = 1.0 if cast else 448.0 / float(2.0 ** np.float32(8.807))
    np.testing.assert_allclose(out, 6.0 * weight, rtol=4e-3, atol=0)


def test_sageattn_vc_fp8_end_to_end_and_layouts():
    from sageattention_local import sageattn_vc_fp8
    from sageattention_local.vc_fp8 import forward_prepared, prepare
    q, k, v = make_qkv(1, 2, 1000, 1500, 128, torch.bfloat16, seed=5)
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    for cast in (True, False):
        _print_case("sageattn_vc_fp8", cast)
        st = prepare(qd, kd, vd, expcast=cast)
        ost = o.prepare_fp8(bits(q), bits(k), bits(v), expcast=cast)
        for key in ("q", "k", "qs", "ks", "vs"):
            np.testing.assert_array_equal(st[key].cpu().numpy(), ost[key])
        np.testing.assert_array_equal(storage_to_logical(st["v"], vcx.value_token()), ost["v"])
        out = forward_prepared(st)
        dump, codes = vcx.forward_fp8(st["q"], st["k"], st["v"], st["qs"], st["ks"], st["vs"], cast,
                                      st["output_type"], st["scale"], p_rows=(0, 1000))
        assert torch.equal(dump, out)  # the diagnostic variant computes the same output bits
        got = out.float().cpu().numpy()
        err, bound = output_bound(got, _expected_from_codes(ost, codes.cpu().numpy(), cast))
        assert np.all(err <= bound)
        assert cosine(got, o.reference(ost, affine=cast)) >= 0.9999
        full = sageattn_vc_fp8(qd, kd, vd, expcast=cast)
        assert torch.equal(full, out)
        nhd = sageattn_vc_fp8(*(x.transpose(1, 2).contiguous() for x in (qd, kd, vd)), tensor_layout="NHD",
                              expcast=cast)
        assert torch.equal(nhd.transpose(1, 2), out)


def test_fp8_kernel_resources_and_rejections():
    from sageattention_local.vc_fp8 import fp8_kernel_resources, forward_prepared
    res = fp8_kernel_resources(1, 128)
    assert set(res) == {"fp8_control", "fp8_expcast"}
    assert all(r["scratch_bytes_per_lane"] == 0 and r["vgprs"] <= 256 for r in res.values())
    with pytest.raises(ValueError, match="FP8 block"):
        forward_prepared({"qk_format": "int8"})
    with pytest.raises(ValueError, match="FP8 block"):
        forward_prepared({"qk_format": "fp8_block", "block_values": True})
    q8 = torch.zeros(1, 1, 65, 64, dtype=torch.uint8, device=DEV)
    k8 = torch.zeros(1, 1, 129, 64, dtype=torch.uint8, device=DEV)
    v8 = torch.zeros(1, 1, 64, 256, dtype=torch.uint8, device=DEV)
    qs, ks, vs = (torch.ones(s, device=DEV) for s in ((1, 1, 2), (1, 1, 2), (1, 1, 64)))
    with pytest.raises(vcx.VcxError, match="scales"):
        vcx.forward_fp8(q8, k8, v8, qs[..., :1].contiguous(), ks, vs, True, 1, 0.125)
    with pytest.raises(vcx.VcxError, match="int8|E4M3|float8"):
        vcx.forward_fp8(q8.view(torch.int8), k8, v8, qs, ks, vs, True, 1, 0.125)


# ------------------------------------------------------------------ the reference's vc27 gates

GATE_ATTN = [(1, 1), (17, 63), (63, 127), (64, 128), (65, 129), (127, 255), (128, 256), (129, 257), (193, 513)]


def _relative_rmse(actual, expected):
    d = np.asarray(actual, np.float64) - np.asarray(expected, np.float64)
    return float(np.sqrt((d ** 2).mean()) / max(np.sqrt((np.asarray(expected, np.float64) ** 2).mean()), 1e-12))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
def test_fp8_attention_gate_all_rows(D, dt):
    # scripts/validate_fp8_qk.py:128-155: every shape and both probability paths within 1 %
    # relative RMSE of the decoded-payload oracle (here, as everywhere, also the elementwise
    # bound against the attention the kernel's own P bytes define); the public API and its
    # NHD layout give the same bits as forward_prepared.
    from sageattention_local import sageattn_vc_fp8
    from sageattention_local.vc_fp8 import forward_prepared, prepare
    gen = torch.Generator().manual_seed(2702 + D)
    for nq, nk in GATE_ATTN:
        q = torch.randn(2, 2, nq, D, generator=gen).to(dt)
        k = torch.randn(2, 2, nk, D, generator=gen).to(dt)
        v = torch.randn(2, 2, nk, D, generator=gen).to(dt)
        qd, kd, vd = (x.to(DEV) for x in (q, k, v))
        ost = o.prepare_fp8(bits(q), bits(k), bits(v), dtype=dtype_name(dt))
        for cast in (False, True):
            _print_case("fp8 gate", nq, nk, D, dt, cast)
            st = prepare(qd, kd, vd, expcast=cast)
            out = forward_prepared(st)
            ost["expcast"] = cast
            eout = o.reference(ost, affine=cast)
            got = out.float().cpu().numpy()
            assert np.isfinite(got).all()
            assert _relative_rmse(got, eout) <= 0.01
            _, codes = vcx.forward_fp8(st["q"], st["k"], st["v"], st["qs"], st["ks"], st["vs"], cast,
                                       st["output_type"], st["scale"], p_rows=(0, nq))
            err, bound = output_bound(got, _expected_from_codes(ost, codes.cpu().numpy(), cast))
            assert np.all(err <= bound)
            assert torch.equal(sageattn_vc_fp8(qd, kd, vd, expcast=cast), out)
            nhd = sageattn_vc_fp8(qd.transpose(1, 2), kd.transpose(1, 2), vd.transpose(1, 2), tensor_layout="NHD",
                                  expcast=cast)
            assert torch.equal(nhd.transpose(1, 2), out)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
def test_fp8_known_constant_values_and_zero_channels(D, dt):
    # scripts/validate_fp8_qk.py:156-170: zero Q/K, V = (channel % 8) / 8 (every 8th channel
    # zero) or all zero: finite payloads, and the output is V's constant row.
    from sageattention_local import sageattn_vc_fp8
    from sageattention_local.vc_fp8 import prepare
    q = torch.zeros(1, 2, 65, D, device=DEV, dtype=dt)
    for nk in (1, 129, 257):
        k = torch.zeros(1, 2, nk, D, device=DEV, dtype=dt)
        for all_zero in (False, True):
            _print_case("fp8 known constant", D, dt, nk, all_zero)
            v = (torch.arange(D, device=DEV, dtype=dt).remainder(8).view(1, 1, 1, D).expand_as(k).contiguous() / 8)
            if all_zero:
                v.zero_()
            st = prepare(q, k, v)
            for name in ("qs", "ks", "vs"):
                assert torch.isfinite(st[name]).all(), name
            for name in ("q", "k", "v"):
                assert torch.isfinite(st[name].view(torch.float8_e4m3fn).float()).all(), name
            for cast in (False, True):
                out = sageattn_vc_fp8(q, k, v, expcast=cast)
                assert torch.isfinite(out).all()
                torch.testing.assert_close(out, v[:, :, :1].expand_as(out), rtol=0.004, atol=0.002)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
def test_fp8_value_zero_channels_on_a_side_stream(D, dt):
    # scripts/validate_fp8_qk.py:85-122 and tests/test_fp8_zero_values.py: zero channels get a
    # zero scale and zero bytes, every other scale is amax/448, on a non-default stream.
    gen = torch.Generator().manual_seed(27101)
    tok = vcx.value_token()
    for n in (1, 128, 129, 257, 4097):
        for kind in ("mixed_random", "mixed_constant", "all_zero"):
            _print_case("fp8 V zero channels", D, dt, n, kind)
            v = torch.randn(2, 3, n, D, generator=gen).to(dt)
            if kind == "mixed_constant":
                v.copy_(torch.arange(D, dtype=dt).remainder(8).view(1, 1, 1, D) / 8)
            if kind == "all_zero":
                v.zero_()
            v[..., ::8] = 0
            vd = v.to(DEV)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                v8, vs, _ = vcx.prepare_v(vd)
            torch.cuda.current_stream().wait_stream(side)
            logical = storage_to_logical(v8, tok)
            ev8, evs = o.per_channel_fp8(bits(v), None, dtype_name(dt))
            np.testing.assert_array_equal(logical, ev8)
            np.testing.assert_array_equal(vs.cpu().numpy(), evs)
            amax = v.float().abs().amax(2).numpy()
            zero = amax == 0
            assert np.all(vs.cpu().numpy()[zero] == 0)
            assert np.count_nonzero(logical[zero]) == 0
            np.testing.assert_allclose(vs.cpu().numpy(), amax / 448, rtol=2e-7, atol=0)
