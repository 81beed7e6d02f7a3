"""Pins of the CPU oracle (oracle/vc_oracle.c) against the reference's known answers,
golden vectors, closed forms and library routines. CPU only.

Each test names the reference file:line whose known answer it reproduces, or the
independent check it relies on (torch's E4M3 cast, exact rational sums, an FP64
Lloyd written differently from the oracle, the Triton quantizer's own outputs).
"""
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import (FOLD_CODE_FOLDED, FOLD_CODE_UNFUSED, FOLD_K, FOLD_KS, FOLD_Q, FOLD_QS, bits,
                     folded_encode_payload, make_qkv)
from oracle import vc_oracle as o

GOLDEN = Path(__file__).resolve().parent / "golden" / "int8_per_thread.npz"


# ------------------------------------------------------------------ ExpCast / E4M3

def test_expcast_known_answers_core():
    # tests/test_core.py:17-22 of the reference (paper worked example included).
    u = torch.tensor([0.0, -1.0, -1.6, -8.0, -14.0, -100.0, -float("inf")])
    codes = o.expcast_codes((u / math.log2(math.e)).numpy())
    assert codes.tolist() == [120, 112, 107, 56, 8, 0, 0]
    assert o.e4m3_decode(codes).tolist() == [256, 128, 88, 1, 2 ** -6, 0, 0]


def test_expcast_known_answers_sage_vc():
    # tests/test_sage_vc.py:22-25 of the reference.
    codes = o.expcast_codes(np.array([-np.inf, -20.0, 0.0, 1.0], np.float32))
    assert codes.tolist() == [0, 0, 120, 120]
    assert o.e4m3_decode(codes).tolist() == [0.0, 0.0, 256.0, 256.0]


def test_expcast_paper_example():
    # tests/test_paper_expcast.py:38-44: -1.60/log2(e) -> 107 -> 88.0
    shifted = np.float32(torch.tensor(-1.60 / 1.4426950408889634).item())
    c = o.expcast_codes(np.array([shifted], np.float32))
    assert c[0] == 107 and o.e4m3_decode(c)[0] == 88.0


def test_expcast_single_rounding_fma_against_exact_arithmetic():
    # The encoder is RNE(fl32(x*A + B)) with ONE rounding of the exact x*A+B.
    # Check against exact rational arithmetic on values spread over the domain,
    # including the reference sweep points (scripts/validate_sage_vc.py:22-24).
    A, B = Fraction(float(np.float32(11.541560173034668))), Fraction(float(np.float32(119.6500015258789)))
    xs = np.concatenate([np.linspace(-15, 1, 4001, dtype=np.float32), np.array([-20.0, 0.0], np.float32)])
    codes = o.expcast_codes(xs)
    for x, c in zip(xs.tolist(), codes.tolist()):
        exact = Fraction(x) * A + B
        f = float(np.float32(float(exact)))  # round exact value once to fp32 (RN via double: exact fits 2*24+ bits)
        # float(exact) rounds to double first; recheck the tie case exactly
        v = Fraction(f)
        expect = min(120, max(0, round(v)))  # Python round: half to even, exact on Fractions
        assert c == expect, (x, c, expect)


def test_e4m3_decode_closed_form_all_codes():
    # tests/test_core.py:89-91 numpy decode formula, all positive codes below NaN.
    code = np.arange(0, 127, dtype=np.uint8)
    exponent, mantissa = code >> 3, code & 7
    values = np.where(exponent == 0, mantissa * 2.0 ** -9, (1 + mantissa / 8) * 2.0 ** (exponent.astype(int) - 7))
    np.testing.assert_array_equal(o.e4m3_decode(code), values.astype(np.float32))
    np.testing.assert_array_equal(o.e4m3_decode(code | 0x80), -values.astype(np.float32))
    assert np.isnan(o.e4m3_decode(np.array([0x7F, 0xFF], np.uint8))).all()


def test_e4m3_encode_matches_torch_cast_and_roundtrips():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * 40,
                        (rng.random(100000).astype(np.float32) - 0.5) * 0.05,
                        np.array([0.0, -0.0, 448.0, -448.0, 1e-30, -1e-30], np.float32)])
    # torch's CPU cast does not saturate (F7), so clamp first, as the kernels do.
    ref = torch.from_numpy(np.clip(x, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(o.e4m3_encode(x), ref)
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    np.testing.assert_array_equal(o.e4m3_encode(o.e4m3_decode(codes)), codes)
    # midpoints between neighbours round to the even code; saturation above 448
    for c in range(1, 0x7E):
        lo, hi = o.e4m3_decode(np.array([c, c + 1], np.uint8))
        mid = np.float32((np.float64(lo) + np.float64(hi)) / 2)
        assert o.e4m3_encode(np.array([mid], np.float32))[0] == (c if c % 2 == 0 else c + 1)
    assert o.e4m3_encode(np.array([500.0, 1e30, np.inf], np.float32)).tolist() == [0x7E, 0x7E, 0x7E]


def test_cvt_u8_model():
    x = np.array([-np.inf, -1.0, -0.4, 0.5, 1.5, 2.5, 119.5, 120.49, 254.5, 255.6, 1e9, np.nan], np.float32)
    assert o.cvt_u8(x).tolist() == [0, 0, 0, 0, 2, 2, 120, 120, 254, 255, 255, 0]


def test_value_permutation_known_answer():
    # tests/test_sage_vc.py:26-28 of the reference.
    perm = o.value_permutation(256)
    assert perm[:16].tolist() == [0, 1, 4, 5, 8, 9, 12, 13, 2, 3, 6, 7, 10, 11, 14, 15]
    assert sorted(perm.tolist()) == list(range(256))


# ------------------------------------------------------------------ fixed-order sums

def test_tile_tree_sum_is_exact_when_representable_and_order_sensitive_otherwise():
    rng = np.random.default_rng(1)
    x = rng.integers(-1000, 1000, 128).astype(np.float64) / 64
    assert o.tile_tree_sum(x) == float(sum(Fraction(v) for v in x))
    # A case where order matters: the documented tree pairs key kk with kk^1 first.
    y = np.zeros(128)
    y[0], y[1], y[16] = 1e16, 1.0, -1e16   # kk=0 chain: 1e16 + (-1e16) = 0, then + a[1] = 1
    assert o.tile_tree_sum(y) == 1.0


# ------------------------------------------------------------------ INT8 quantizer

def test_int8_quantizer_matches_reference_triton_golden_vectors():
    # Vectors written by tests/golden/make_int8_vectors.py from the reference's
    # own per_thread_int8 (quant_per_thread.py:154-204) under TRITON_INTERPRET=1.
    z = np.load(GOLDEN)
    cases = sorted({k.split("_")[0] for k in z.files})
    assert len(cases) == 4
    for c in cases:
        B, H, Nq, Nk, D, bf, _ = z[f"{c}_meta"].tolist()
        dt = "bfloat16" if bf else "float16"
        q8, qs = o.quant_q(z[f"{c}_q"], dt)
        k8, ks = o.quant_k(z[f"{c}_k"], z[f"{c}_km"].reshape(B, H, D), None, dt)
        np.testing.assert_array_equal(q8, z[f"{c}_q8"])
        np.testing.assert_array_equal(qs.view(np.uint32), z[f"{c}_qs"].view(np.uint32))
        np.testing.assert_array_equal(k8, z[f"{c}_k8"])
        np.testing.assert_array_equal(ks.view(np.uint32), z[f"{c}_ks"].view(np.uint32))


def test_int8_quantizer_invariants():
    q, k, _ = make_qkv(1, 2, 193, 300, 64, seed=5)
    q8, qs = o.quant_q(bits(q))
    assert np.abs(q8.astype(int)).max() <= 127
    qf = q.float().numpy()
    rows = np.arange(193)
    sidx = (rows // 16) * 8 + rows % 8
    s = qs[:, :, sidx][..., None]
    assert np.all(np.abs(qf - q8 * s) <= s / 2 * (1 + 1e-5) + 1e-12)
    # the element of largest magnitude of each group maps to +-127
    g = qf[0, 0]
    for blk in range(0, 193, 16):
        for t in range(8):
            grp = [r for r in (blk + t, blk + t + 8) if r < 193]
            if not grp:
                continue
            vals = g[grp]
            i = np.unravel_index(np.abs(vals).argmax(), vals.shape)
            assert abs(int(q8[0, 0][grp][i])) == 127
    # padded groups (rows >= N) get the 1e-7 floor
    assert qs[0, 0, -1] == np.float32(np.float32(0.0) / np.float32(127.0) + np.float32(1e-7))


# ------------------------------------------------------------------ K mean

def test_k_mean_exact_and_within_torch_mean():
    _, k, _ = make_qkv(2, 2, 8, 1000, 128, seed=7)
    km = o.k_mean(bits(k))
    kf = k.double().numpy()
    exact = np.float32(kf.sum(axis=2) / 1000)  # exact here: all values sum without rounding in fp64
    assert np.array_equal(km, bits(torch.from_numpy(exact).to(torch.bfloat16)))
    torch_mean = k.mean(dim=2).float().numpy()   # the reference's formula (vc.py:158)
    ours = torch.from_numpy(km.view(np.int16)).view(torch.bfloat16).float().numpy()
    ulp = np.abs(torch_mean) * 2 ** -7 + 1e-30
    assert np.all(np.abs(ours - torch_mean) <= ulp)


# ------------------------------------------------------------------ V quantizers

def test_v_channel_matches_torch_formula_and_invariants():
    _, _, v = make_qkv(1, 2, 1, 300, 64, seed=9)
    v[0, 1, :, 5] = 0  # a zero channel
    v8, vs = o.per_channel_fp8(bits(v))
    vf = v.float()
    amax = vf.abs().amax(dim=2)
    r = torch.tensor(448.0) / amax                       # IEEE fp32 division
    expect = (vf * r.unsqueeze(2)).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    expect[0, 1, :, 5] = 0
    got = v8[..., :300].transpose(0, 1, 3, 2)
    np.testing.assert_array_equal(got, expect.numpy())
    assert np.all(v8[..., 300:] == 0)
    np.testing.assert_array_equal(vs, (amax / torch.tensor(448.0)).numpy())
    assert vs[0, 1, 5] == 0
    # the channel maximum encodes to 448 (0x7E, or 0xFE if negative)
    idx = vf.abs().argmax(dim=2)
    for h in range(2):
        for d in range(64):
            if d == 5 and h == 1:
                continue
            assert v8[0, h, d, idx[0, h, d]] & 0x7F == 0x7E


@pytest.mark.parametrize("n", [1, 127, 128, 129, 257])
@pytest.mark.parametrize("channel", [True, False])
def test_v_smoothing_reference_tolerances(n, channel):
    # scripts/validate_sage_vc.py:29-65 of the reference: unequal block means and
    # scales, constant channels; scale rtol 2e-5, means*vs rtol 8e-4, residual
    # bound 0.063|r| + vs/512 + 3e-6, zero padding.
    torch.manual_seed(339)
    v = torch.randn(2, 2, n, 64)
    for t, begin in enumerate(range(0, n, 128)):
        v[:, :, begin:begin + 128] = v[:, :, begin:begin + 128] * (t + 1) + t * 3
    v[..., 0] = 1.5
    v[..., 1] = -2.0
    v = v.to(torch.bfloat16)
    v8, vs, means = o.prepare_values(bits(v), channel_scale=channel)
    unpacked = torch.from_numpy(o.e4m3_decode(v8)).transpose(-1, -2)
    meansf = torch.from_numpy(means.view(np.float16).astype(np.float32))
    blocks = []
    for begin in range(0, n, 128):
        rows = v[:, :, begin:begin + 128].float()
        mean = rows.mean(2)
        residual = rows - mean.unsqueeze(2)
        blocks.append((mean, residual, residual.abs().amax(2)))
    vs_t = torch.from_numpy(vs)
    if channel:
        peak = torch.stack([b[2] for b in blocks]).amax(0)
        mean_peak = torch.stack([b[0].abs() for b in blocks]).amax(0)
        expected_scale = torch.maximum(torch.where(peak > 0, peak / 448., 1.), mean_peak / 65504.)
        torch.testing.assert_close(vs_t, expected_scale, rtol=2e-5, atol=1e-7)
    for t, (mean, residual, peak) in enumerate(blocks):
        scale = vs_t if channel else vs_t[:, :, t]
        if not channel:
            expected_scale = torch.maximum(torch.where(peak > 0, peak / 448., 1.), mean.abs() / 65504.)
            torch.testing.assert_close(scale, expected_scale, rtol=2e-5, atol=1e-7)
        torch.testing.assert_close(meansf[:, :, t] * scale, mean, rtol=8e-4, atol=2e-6)
        decoded = unpacked[:, :, t * 128:t * 128 + residual.shape[2]]
        err = (decoded * scale.unsqueeze(2) - residual).abs()
        bound = residual.abs() * .063 + scale.unsqueeze(2) / 512 + 3e-6
        assert torch.all(err <= bound)
    if n % 128:
        assert np.count_nonzero(v8[..., n:]) == 0


@pytest.mark.parametrize("n", [1, 129, 4097])
def test_v_smoothing_constant_blocks_and_large_means(n):
    # tests/test_sage_vc_preprocess_cuda.py:48-65: constants per block/channel above
    # the FP16 range; residual bytes all zero; means*scale restore the constants.
    v = torch.zeros(2, 3, n, 64)
    for t, start in enumerate(range(0, n, 128)):
        v[:, :, start:start + 128] = (torch.arange(64) - 31) * (t + 1) * 10000.
    v = v.to(torch.bfloat16)
    v8, vs, means = o.prepare_values(bits(v))
    restored = torch.from_numpy(means.view(np.float16).astype(np.float32)) * torch.from_numpy(vs).unsqueeze(2)
    assert np.isfinite(vs).all() and np.isfinite(means.view(np.float16)).all()
    assert np.count_nonzero(o.e4m3_decode(v8)) == 0
    torch.testing.assert_close(restored, v[:, :, ::128].float(), rtol=5e-4, atol=1e-6)


def test_v_smoothing_reduction_beyond_one_warp():
    # tests/test_sage_vc_preprocess_cuda.py:68-80 (fp32 input there; bf16 here).
    torch.manual_seed(919)
    v = torch.randn(2, 3, 4353, 128) * .01
    v[:, :, 4224:4352] *= 1000
    v[:, :, -1] = 90000
    v = v.to(torch.bfloat16)
    v8, vs, means = o.prepare_values(bits(v))
    vf = v.float()
    blocks = [vf[:, :, i:i + 128] for i in range(0, vf.shape[2], 128)]
    raw_means = torch.stack([x.mean(2) for x in blocks], 2)
    peaks = torch.stack([(x - x.mean(2, keepdim=True)).abs().amax(2) for x in blocks], 2).amax(2)
    expected = torch.maximum(peaks / 448, raw_means.abs().amax(2) / 65504)
    torch.testing.assert_close(torch.from_numpy(vs), expected, rtol=2e-5, atol=1e-7)
    m = torch.from_numpy(means.view(np.float16).astype(np.float32))
    torch.testing.assert_close(m * torch.from_numpy(vs).unsqueeze(2), raw_means, rtol=1e-3, atol=1e-5)


# ------------------------------------------------------------------ grouping

def fp64_lloyd(v, clusters, iterations):
    """The reference's independent FP64 oracle (tests/test_sage_vc_grouping_cuda.py:8-23)."""
    count = min(clusters, v.shape[2])
    ids = torch.linspace(0, v.shape[2] - 1, count).long()
    x = v.double()
    centers = x.index_select(2, ids)
    for step in range(iterations):
        distances = (x.unsqueeze(-2) - centers.unsqueeze(2)).square().sum(-1)
        labels = distances.argmin(-1)
        if step + 1 < iterations:
            centers = torch.stack([
                torch.where((labels == c).sum(-1, keepdim=True) > 0,
                            (x * (labels == c).unsqueeze(-1)).sum(2) / (labels == c).sum(-1, keepdim=True).clamp_min(1),
                            centers[:, :, c]) for c in range(count)], 2)
    return labels, centers


def fp64_lloyd_from(v, centers, iterations):
    """The same FP64 Lloyd from given initial centers, one cluster at a time (bounded memory);
    also returns the update of the final labels (the warm start core.py:153-171 caches)."""
    x = v.double()
    centers = centers.double()
    count = centers.shape[2]

    def update(labels, centers):
        out = []
        for c in range(count):
            m = (labels == c)
            n_c = m.sum(-1, keepdim=True)
            out.append(torch.where(n_c > 0, (x * m.unsqueeze(-1)).sum(2) / n_c.clamp_min(1), centers[:, :, c]))
        return torch.stack(out, 2)

    for step in range(iterations):
        dist = torch.stack([(x - centers[:, :, c:c + 1]).square().sum(-1) for c in range(count)], -1)
        labels = dist.argmin(-1)
        if step + 1 < iterations:
            centers = update(labels, centers)
    return labels, centers, update(labels, centers)


@pytest.mark.parametrize("n,clusters,iterations", [(2049, 16, 2), (1000, 64, 3), (600, 256, 2), (100, 256, 2)])
def test_grouping_many_clusters_matches_independent_fp64_lloyd(n, clusters, iterations):
    # the reference's public grouping serves up to 256 clusters (pybind.cpp:6-44, legacy path)
    torch.manual_seed(17 + n)
    v = torch.randn(2, 2, n, 64).to(torch.bfloat16)
    perm, labels, centers, nxt = o.group_values(bits(v), clusters, iterations, return_next=True)
    count = min(clusters, n)
    ids = torch.linspace(0, n - 1, count).long()
    elabels, ecenters, enext = fp64_lloyd_from(v, v.float().index_select(2, ids), iterations)
    np.testing.assert_array_equal(labels, elabels.numpy())
    np.testing.assert_allclose(centers, ecenters.numpy(), rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(nxt, enext.numpy(), rtol=2e-5, atol=2e-6)
    np.testing.assert_array_equal(perm, elabels.argsort(dim=-1, stable=True).numpy())


@pytest.mark.parametrize("clusters", [8, 16])
def test_grouping_warm_start_matches_independent_fp64_lloyd(clusters):
    # a LayoutCache refresh reruns grouping from the cached centers (src/vc_attention/core.py:216-221)
    torch.manual_seed(3)
    v0 = torch.randn(1, 3, 700, 128).to(torch.bfloat16)
    v1 = (v0.float() + 0.3 * torch.randn(1, 3, 700, 128)).to(torch.bfloat16)
    _, _, _, cached = o.group_values(bits(v0), clusters, 2, return_next=True)
    perm, labels, centers, nxt = o.group_values(bits(v1), clusters, 2, centers_in=cached, return_next=True)
    elabels, ecenters, enext = fp64_lloyd_from(v1, torch.from_numpy(cached), 2)
    np.testing.assert_array_equal(labels, elabels.numpy())
    np.testing.assert_allclose(centers, ecenters.numpy(), rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(nxt, enext.numpy(), rtol=2e-5, atol=2e-6)
    np.testing.assert_array_equal(perm, elabels.argsort(dim=-1, stable=True).numpy())
    # one iteration from the cached centers is a single assignment to exactly those centers
    _, l1, c1 = o.group_values(bits(v1), clusters, 1, centers_in=cached)
    np.testing.assert_array_equal(c1.view(np.uint32), cached.view(np.uint32))
    # the warm start changes the result relative to the linspace start (it is really used)
    _, lcold, _ = o.group_values(bits(v1), clusters, 2)
    assert not np.array_equal(lcold, labels)


@pytest.mark.parametrize("n,clusters,iterations", [(1, 8, 2), (7, 8, 1), (127, 3, 3), (128, 1, 2), (129, 8, 2), (2049, 8, 2)])
def test_grouping_matches_independent_fp64_lloyd(n, clusters, iterations):
    torch.manual_seed(211 + n)
    v = torch.randn(2, 2, n, 64).to(torch.bfloat16)
    perm, labels, centers = o.group_values(bits(v), clusters, iterations)
    expected, expected_centers = fp64_lloyd(v, clusters, iterations)
    np.testing.assert_array_equal(labels, expected.numpy())
    np.testing.assert_allclose(centers, expected_centers.numpy(), rtol=2e-5, atol=2e-6)
    np.testing.assert_array_equal(perm, expected.argsort(dim=-1, stable=True).numpy())


def test_grouping_known_answers():
    # scripts/validate_sage_vc.py:66-76: labels [2,0,1,2,1,0] -> perm [0,3,2,4,1,5]
    x = torch.tensor([2, 0, 1, 2, 1, 0], dtype=torch.float32)
    v = x.view(1, 1, 6, 1).expand(2, 2, 6, 64).contiguous().to(torch.bfloat16)
    perm, labels, _ = o.group_values(bits(v), 3, 2)
    for row in perm.reshape(-1, 6):
        assert row.tolist() == [0, 3, 2, 4, 1, 5]
    # tests/test_sage_vc_grouping_cuda.py:122-133: constant V -> label 0, identity, centers kept
    v = torch.full((2, 3, 257, 128), 2.0).to(torch.bfloat16)
    for it in (1, 2, 3):
        perm, labels, centers = o.group_values(bits(v), 8, it)
        assert labels.sum() == 0
        np.testing.assert_array_equal(perm, np.broadcast_to(np.arange(257), (2, 3, 257)))
        assert (centers == 2).all()


def test_linspace_ids_match_torch():
    for n in list(range(1, 300)) + [37741, 32760, 75482]:
        for count in range(1, 9):
            c = min(count, n)
            assert o.linspace_ids(n, c).tolist() == torch.linspace(0, n - 1, c).long().tolist()


# ------------------------------------------------------------------ attention oracle known answers

def payload(nq, nk, block_values, dim=64, expcast=True):
    """The reference's fixed payload (tests/test_sage_vc.py:31-39)."""
    tiles = (nk + 127) // 128
    return {"q": np.zeros((1, 1, nq, dim), np.int8), "k": np.zeros((1, 1, nk, dim), np.int8),
            "v": np.zeros((1, 1, dim, tiles * 128), np.uint8),
            "qs": np.ones((1, 1, ((nq + 63) // 64) * 32), np.float32), "ks": np.ones((1, 1, tiles * 4), np.float32),
            "vs": np.ones((1, 1, tiles, dim), np.float32) if block_values else np.ones((1, 1, dim), np.float32),
            "means": np.zeros((1, 1, tiles, dim), np.uint16) if block_values else None,
            "expcast": expcast, "block_values": block_values, "scale": dim ** -0.5}


def f16bits(values):
    return np.asarray(values, np.float16).view(np.uint16)


# The Sage FP8 control path (expcast=False) divides FP8(P) by the unrounded exp2 mass, so
# a single or uniform key carries the weight 448 / 2^8.807f (tests/test_sage_vc.py:62-63,
# scripts/validate_sage_vc.py:174-178).
CONTROL_WEIGHT = 448.0 / 2.0 ** float(np.float32(8.807))


@pytest.mark.parametrize("expcast", [False, True])
def test_block_mean_restoration_and_tail_weight_known_answer(expcast):
    # tests/test_sage_vc.py:42-49
    s = payload(65, 257, True, expcast=expcast)
    s["means"][0, 0] = f16bits(np.array([1., -2., 6.])[:, None] * np.ones((1, 64)))
    s["vs"][0, 0] = np.array([2., 3., 4.])[:, None]
    out = o.reference(s)
    np.testing.assert_allclose(out, (128 * 2 + 128 * (-6) + 24) / 257, rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("block_values", [False, True])
@pytest.mark.parametrize("expcast", [False, True])
def test_single_key_preserves_nonzero_value(block_values, expcast):
    # tests/test_sage_vc.py:52-65: weight 1 (ExpCast) or 448 / 2^8.807f (control).
    s = payload(17, 1, block_values, expcast=expcast)
    data = (np.arange(64) % 9 - 4).astype(np.float32)
    s["v"][0, 0, :, 0] = o.e4m3_encode(data)
    s["vs"][...] = 0.125
    if block_values:
        s["means"][...] = f16bits(2.0)
    out = o.reference(s)
    weight = 1.0 if expcast else CONTROL_WEIGHT
    expected = (data * weight + (2 if block_values else 0)) * 0.125
    np.testing.assert_allclose(out, np.broadcast_to(expected, out.shape), rtol=1e-6, atol=1e-6)


def test_query_sampling_keeps_original_scale_indices():
    # tests/test_sage_vc.py:68-79
    s = payload(129, 129, False)
    rng = np.random.default_rng(778)
    s["q"][...] = rng.integers(-3, 4, s["q"].shape)
    s["k"][...] = rng.integers(-3, 4, s["k"].shape)
    s["qs"][...] = rng.uniform(0.1, 0.3, s["qs"].shape)
    s["ks"][...] = rng.uniform(0.2, 0.5, s["ks"].shape)
    s["v"][...] = o.e4m3_encode(rng.standard_normal(s["v"].shape).astype(np.float32))
    ids = [0, 7, 8, 15, 16, 63, 64, 128]
    all_rows, all_codes = o.reference(s, return_codes=True)
    sampled, codes = o.reference(s, query_indices=ids, return_codes=True)
    np.testing.assert_array_equal(sampled, all_rows[:, :, ids])
    np.testing.assert_array_equal(codes, all_codes[:, :, ids])


@pytest.mark.parametrize("expcast", [False, True])
def test_channel_scale_epilogue_matches_expanded_per_tile_scales(expcast):
    # tests/test_sage_vc.py:82-95
    rng = np.random.default_rng(918)
    s = payload(65, 257, True, expcast=expcast)
    s["q"][...] = rng.integers(-4, 5, s["q"].shape)
    s["k"][...] = rng.integers(-4, 5, s["k"].shape)
    s["qs"][...] = .1
    s["ks"][...] = .15
    s["v"][...] = o.e4m3_encode(rng.standard_normal(s["v"].shape).astype(np.float32))
    s["means"][...] = f16bits(rng.standard_normal(s["means"].shape))
    scales = np.linspace(.01, 1, 64, dtype=np.float32).reshape(1, 1, 64)
    channel = dict(s, vs=scales)
    old = dict(s, vs=np.ascontiguousarray(np.broadcast_to(scales[:, :, None], (1, 1, 3, 64))))
    np.testing.assert_allclose(o.reference(channel), o.reference(old), rtol=5e-5, atol=1e-6)


@pytest.mark.parametrize("expcast", [False, True])
def test_shared_scale_nonzero_mean_known_answer(expcast):
    # tests/test_sage_vc.py:98-105
    s = payload(65, 257, True, expcast=expcast)
    s["vs"] = np.full((1, 1, 64), .25, np.float32)
    s["means"][0, 0] = f16bits(np.array([8., -24., 96.])[:, None] * np.ones((1, 64)))
    out = o.reference(s)
    np.testing.assert_allclose(out, (128 * 2 - 128 * 6 + 24) / 257, rtol=2e-6, atol=1e-6)


def test_expcast_codes_agree_with_dense_numpy_formula_one_tile():
    # tests/test_core.py:80-93: codes from clip(rint(8u + 119.65)) with u in double;
    # the oracle's fp32 RN logits/subtraction/FMA may differ only at rounding ties.
    rng = np.random.default_rng(3)
    s = payload(19, 35, False, dim=64)
    s["q"][...] = rng.integers(-20, 21, s["q"].shape)
    s["k"][...] = rng.integers(-20, 21, s["k"].shape)
    _, codes = o.reference(s, return_codes=True)
    logits = (s["q"][0, 0].astype(np.float64) @ s["k"][0, 0].T.astype(np.float64)) * np.float32(64 ** -0.5)
    u = (logits - logits.max(-1, keepdims=True)) * math.log2(math.e)
    ref = np.clip(np.rint(8 * u + 119.65), 0, 120).astype(np.uint8)
    got = codes[0, 0, :, :35]
    assert np.mean(got == ref) > 0.99 and np.abs(got.astype(int) - ref).max() <= 1
    assert np.all(codes[0, 0, :, 35:] == 0)


@pytest.mark.parametrize("expcast", [False, True])
def test_uniform_attention_equals_decoded_value_mean(expcast):
    # scripts/validate_sage_vc.py:161-182: q = k = 0; weight 1 (ExpCast) or 448 / 2^8.807f.
    rng = np.random.default_rng(4)
    s = payload(65, 513, False, expcast=expcast)
    s["v"][..., :513] = o.e4m3_encode((np.arange(513) / 128 - 2).astype(np.float32))[None, None, None, :]
    s["vs"][...] = np.linspace(0.5, 1.5, 64)
    dec = o.e4m3_decode(s["v"][0, 0, :, :513]).astype(np.float64)
    expected = dec.mean(-1) * s["vs"][0, 0] * (1.0 if expcast else CONTROL_WEIGHT)
    out, codes = o.reference(s, return_codes=True)
    np.testing.assert_allclose(out[0, 0], np.broadcast_to(expected, (65, 64)), rtol=1e-6, atol=1e-6)
    # every valid key gets the largest byte of its path, padding keys get 0
    assert np.all(codes[..., :513] == (120 if expcast else 0x7E)) and np.all(codes[..., 513:] == 0)
    del rng


def _control_case(seed, nq=24, nk=300, dim=64):
    rng = np.random.default_rng(seed)
    s = payload(nq, nk, False, dim=dim, expcast=False)
    s["q"][...] = rng.integers(-60, 61, s["q"].shape)
    s["k"][...] = rng.integers(-60, 61, s["k"].shape)
    s["qs"][...] = rng.uniform(0.04, 0.09, s["qs"].shape)
    s["ks"][...] = rng.uniform(0.04, 0.09, s["ks"].shape)
    s["v"][..., :nk] = o.e4m3_encode(rng.standard_normal((1, 1, dim, nk)).astype(np.float32))
    s["vs"][...] = rng.uniform(0.5, 2.0, s["vs"].shape)
    # exact log2-domain logits of the payload: acc * qs[row] * ks[tile, (key%8)//2] * sm * log2 e
    rows, keys = np.arange(nq), np.arange(nk)
    acc = s["q"][0, 0].astype(np.float64) @ s["k"][0, 0].T.astype(np.float64)
    qsc = s["qs"][0, 0][(rows // 16) * 8 + rows % 8].astype(np.float64)
    ksc = s["ks"][0, 0][(keys // 128) * 4 + (keys % 8) // 2].astype(np.float64)
    lg2 = acc * qsc[:, None] * ksc[None, :] * (dim ** -0.5) * math.log2(math.e)
    return s, lg2


def test_control_bytes_are_e4m3_of_exp2_with_the_fp8_offset():
    # attn_utils.cuh:30,378-386,436-452: the running maximum (over the tiles so far) carries
    # the 8.807 offset, so the largest P of a row is 2^8.807 ~ 448 (byte 0x7E) and
    # P = E4M3(2^(l - running max l + 8.807)). Checked against float64 logits and torch's
    # E4M3 cast; the oracle's fp32 FMAs may differ only next to a rounding midpoint.
    s, lg2 = _control_case(11)
    _, codes = o.reference(s, return_codes=True)
    nk = lg2.shape[1]
    tile_max = np.stack([lg2[:, t:t + 128].max(-1) for t in range(0, nk, 128)], -1)
    running = np.maximum.accumulate(tile_max, axis=-1)
    shifted = lg2 - (running[:, np.arange(nk) // 128] - 8.807)
    want = torch.from_numpy(np.exp2(shifted).astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = codes[0, 0, :, :lg2.shape[1]]
    assert np.mean(got == want) > 0.995 and np.abs(got.astype(int) - want).max() <= 1
    assert np.all(got.max(-1) == 0x7E) and np.all(codes[0, 0, :, lg2.shape[1]:] == 0)


def test_control_output_is_a_base_e_softmax_within_the_fp8_bound():
    # vc_sm90.cu:177 scales by log2 e, so the control path is softmax(logits) @ V with only
    # the E4M3 rounding of P in the numerator: |E4M3(p) - p| <= 2^-4 p + 2^-10 for P in the
    # units of the offset maximum (p <= 448; 2^-10 is half the subnormal quantum).
    s, lg2 = _control_case(12)
    out = o.reference(s)[0, 0].astype(np.float64)
    w = np.exp2(lg2 - lg2.max(-1, keepdims=True) + 8.807)
    dec = o.e4m3_decode(s["v"][0, 0, :, :lg2.shape[1]]).astype(np.float64) * s["vs"][0, 0, :, None]
    exact = (w @ dec.T) / w.sum(-1, keepdims=True)
    bound = ((2.0 ** -4 * w + 2.0 ** -10) @ np.abs(dec.T)) / w.sum(-1, keepdims=True)
    assert np.all(np.abs(out - exact) <= bound + 1e-6)
    # and a base-2 softmax (no log2 e) is far outside that bound
    w2 = np.exp2((lg2 - lg2.max(-1, keepdims=True)) / math.log2(math.e))
    wrong = (w2 @ dec.T) / w2.sum(-1, keepdims=True)
    assert np.mean(np.abs(wrong - exact) > bound) > 0.3


def test_expcast_codes_multi_tile_running_max_and_scale_indices():
    # The P-byte rule of sal/csrc/vc/vc_sm90.cu:288-289,417-418,450,465-482 and
    # vc_math.cuh:268-384, restated here in vectorised float32 numpy (not the oracle's
    # loop): the codes of tile t use the running max over tiles 0..t, tiles before the
    # last round float(acc) * RN(sm * RN(qs*ks)), the last tile rounds (float(acc)*dq)*sm
    # and masks keys >= Nk; qs index (row//16)*8 + row%8, ks index tile*4 + (key%8)//2.
    # Later tiles carry larger logits so that using the global max or a wrong scale
    # index changes many codes. At D=64 sm = 2^-3, so both rounding orders agree here;
    # the last tile's order is pinned at D=128 by the known answer below.
    rng = np.random.default_rng(21)
    nq, nk, dim = 40, 300, 64
    s = payload(nq, nk, False, dim=dim)
    s["q"][...] = rng.integers(-9, 10, s["q"].shape)
    k = rng.integers(-9, 10, s["k"].shape)
    k[..., 128:256, :] = np.clip(k[..., 128:256, :] * 2, -127, 127)
    k[..., 256:, :] = np.clip(k[..., 256:, :] * 3, -127, 127)
    s["k"][...] = k
    s["qs"][...] = rng.uniform(0.02, 0.05, s["qs"].shape).astype(np.float32)
    s["ks"][...] = rng.uniform(0.02, 0.05, s["ks"].shape).astype(np.float32)
    _, codes = o.reference(s, return_codes=True)

    f32 = np.float32
    sm = f32(dim ** -0.5)
    acc = s["q"][0, 0].astype(np.int64) @ s["k"][0, 0].T.astype(np.int64)  # exact int
    rows, keys = np.arange(nq), np.arange(nk)
    qs = s["qs"][0, 0][(rows // 16) * 8 + rows % 8].astype(f32)[:, None]
    ks = s["ks"][0, 0][(keys // 128) * 4 + (keys % 8) // 2].astype(f32)[None, :]
    dq = (qs * ks).astype(f32)
    accf = acc.astype(f32)
    m = np.full((nq, 1), f32(-5e6), f32)
    expected = np.zeros((nq, 384), np.uint8)
    tiles = (nk + 127) // 128
    for t in range(tiles):
        cols = slice(128 * t, min(128 * (t + 1), nk))
        if t < tiles - 1:
            logit = (accf[:, cols] * (sm * dq[:, cols]).astype(f32)).astype(f32)
        else:
            logit = ((accf[:, cols] * dq[:, cols]).astype(f32) * sm).astype(f32)
        m = np.maximum(m, logit.max(-1, keepdims=True))
        u = (logit - m).astype(f32)
        # fmaf(u, A, B): the fp64 product of two floats is exact; one rounding to fp32
        # after the fp64 add (ties at fp32 half-ulps of the sum do not occur here).
        v = (u.astype(np.float64) * np.float64(11.541560173034668) + np.float64(119.6500015258789)).astype(f32)
        expected[:, cols] = np.clip(np.rint(v), 0, 120).astype(np.uint8)
    np.testing.assert_array_equal(codes[0, 0], expected)
    # the running max matters: codes relative to the global max differ in tile 0
    gmax = (accf * (sm * dq).astype(f32)).astype(f32).max(-1, keepdims=True)
    assert np.any(expected[:, :128] != np.clip(np.rint(8 * math.log2(math.e) * (
        (accf[:, :128] * (sm * dq[:, :128]).astype(f32)) - gmax) + 119.65), 0, 120).astype(np.uint8))


@pytest.mark.parametrize("nk", [2, 128, 129, 300])
def test_last_tile_rounding_order_known_answer(nk):
    # sal/csrc/vc/vc_sm90.cu:417-418 (last tile: (acc*dq)*sm) vs :288-289 (acc*(sm*dq)):
    # the same two dot products give byte 96 in the last tile and 97 before it.
    from helpers import ORDER_CODE_LAST, ORDER_CODE_OTHER, rounding_order_payload
    _, codes = o.reference(rounding_order_payload(nk), return_codes=True)
    assert codes[0, 0, 0, 0] == 120
    assert codes[0, 0, 0, 1] == (ORDER_CODE_LAST if nk <= 128 else ORDER_CODE_OTHER)
    assert np.all(codes[0, 0, 0, 2:] == 0)


# ------------------------------------------------------------------ folded ExpCast encode

def _rn32(x):
    """Exact rational -> nearest binary32 (ties to even), as a Fraction."""
    f = np.float32(float(x))
    cands = [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - x), int(np.float32(c).view(np.uint32)) & 1))
    return Fraction(float(best))


def test_folded_encode_known_answer_against_exact_arithmetic():
    # sal/csrc/vc/vc_math.cuh:76-111 (FoldAffine, the reference's default "optimized"/vc15
    # kernel without block values): gain = RN(scale * A), bias = fmaf(-m', A, B),
    # code = sat_u8(RNE(fmaf(float(acc), gain, bias))) with scale = RN(sm * RN(qs * ks)).
    # The unfused code is RNE(fmaf(RN(RN(float(acc) * scale) - m'), A, B)). Both are
    # recomputed here in exact rational arithmetic with one rounding per IEEE step.
    s = folded_encode_payload()
    _, plain = o.reference(s, return_codes=True)
    _, fold = o.reference(s, return_codes=True, affine=True)
    assert plain[0, 0, 0, 96] == FOLD_CODE_UNFUSED and fold[0, 0, 0, 96] == FOLD_CODE_FOLDED
    assert plain[0, 0, 0, 45] == fold[0, 0, 0, 45] == 120
    A, B = Fraction(float(np.float32(11.541560173034668))), Fraction(float(np.float32(119.6500015258789)))
    sm = np.float32(64 ** -0.5)
    acc = {key: int(np.dot(np.int64(FOLD_Q), np.int64(row))) for key, row in FOLD_K.items()}
    scale = {key: np.float32(sm * np.float32(np.float32(FOLD_QS) * np.float32(FOLD_KS[(key % 8) // 2])))
             for key in FOLD_K}
    m = np.float32(np.float32(acc[45]) * scale[45])
    shifted = np.float32(np.float32(np.float32(acc[96]) * scale[96]) - m)
    assert round(_rn32(Fraction(float(shifted)) * A + B)) == FOLD_CODE_UNFUSED
    gain = Fraction(float(np.float32(scale[96] * np.float32(11.541560173034668))))
    bias = _rn32(-Fraction(float(m)) * A + B)
    assert round(_rn32(Fraction(acc[96]) * gain + bias)) == FOLD_CODE_FOLDED


def test_folded_encode_falls_back_per_sixteen_row_group():
    # vc_math.cuh:102-110: if any row of the warp's 16 rows has |m'| > 128 (or a scale
    # underflows / the gain overflows), the whole group uses the unfused encode this tile.
    _, same_group = o.reference(folded_encode_payload(extreme_rows=(3,)), return_codes=True, affine=True)
    assert same_group[0, 0, 0, 96] == FOLD_CODE_UNFUSED
    s = folded_encode_payload(extreme_rows=(19,))
    _, other_group = o.reference(s, return_codes=True, affine=True)
    _, unfused = o.reference(s, return_codes=True)
    assert other_group[0, 0, 0, 96] == FOLD_CODE_FOLDED
    np.testing.assert_array_equal(other_group[0, 0, 16:], unfused[0, 0, 16:])


def test_folded_encode_differs_from_unfused_only_next_to_ties():
    # On N(0,1) inputs the two encodes disagree on a few bytes per million, by one code.
    q, k, v = make_qkv(1, 1, 128, 2048, 128, torch.bfloat16, seed=0)
    st = o.prepare(bits(q), bits(k), bits(v), v_smooth=False, dtype="bfloat16")
    out1, c1 = o.reference(st, return_codes=True)
    out2, c2 = o.reference(st, return_codes=True, affine=True)
    d = np.abs(c1.astype(int) - c2.astype(int))
    assert d.max() <= 1 and np.count_nonzero(d) <= d.size // 50000
    np.testing.assert_allclose(out1, out2, rtol=0, atol=1e-3)
    with pytest.raises(ValueError, match="without block values"):
        o.reference(o.prepare(bits(q), bits(k), bits(v), v_smooth=True, dtype="bfloat16"), affine=True)


# ------------------------------------------------------------------ FP8 block QK (vc27)

def _fp8_quant_reference(x, rows, mean=None):
    # scripts/validate_fp8_qk.py:8-20, restated with torch: per block of `rows` rows the scale
    # is RN(amax/448) (>= 1e-12, IEEE division via float64) and the code RN(x/s) cast to E4M3.
    x = x.float()
    if mean is not None:
        x = x - mean.unsqueeze(2)
    packed, scales = [], []
    for start in range(0, x.shape[2], rows):
        block = x[:, :, start:start + rows]
        scale = (block.abs().amax((-2, -1)).double() / 448).float().clamp_min(1e-12)
        normalized = (block.double() / scale[..., None, None].double()).float()
        packed.append(normalized.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8))
        scales.append(scale)
    return torch.cat(packed, 2).numpy(), torch.stack(scales, 2).numpy()


@pytest.mark.parametrize("nq,nk,dim", [(1, 1, 64), (63, 127, 128), (65, 129, 64), (193, 513, 128)])
def test_fp8_block_quantizer_matches_reference_validation_formula(nq, nk, dim):
    gen = torch.Generator().manual_seed(2701 + nq)
    q = torch.randn(2, 3, nq, dim, generator=gen).to(torch.bfloat16)
    k = torch.randn(2, 3, nk, dim, generator=gen).to(torch.bfloat16)
    k = (k.float() + torch.arange(dim).view(1, 1, 1, -1) / 4).to(torch.bfloat16)  # distinct channel means
    q[:, :, 64:] *= 3
    km = o.k_mean_f32(bits(k))
    exact = k.double().mean(2)
    np.testing.assert_allclose(km, exact.numpy(), rtol=2e-5, atol=1e-5)  # validate_fp8_qk.py:42
    assert np.array_equal(km, exact.float().numpy())  # this definition: the fp64 mean rounded once
    for x, rows, mean in ((q, 64, None), (k, 128, torch.from_numpy(km))):
        codes, scales = o.quant_fp8_block(bits(x), rows, None if mean is None else mean.numpy())
        want_codes, want_scales = _fp8_quant_reference(x, rows, mean)
        np.testing.assert_array_equal(scales, want_scales)
        np.testing.assert_array_equal(codes, want_codes)


def _fp8_payload(nq, nk, dim=64, expcast=True):
    tiles = (nk + 127) // 128
    return {"q": np.zeros((1, 1, nq, dim), np.uint8), "k": np.zeros((1, 1, nk, dim), np.uint8),
            "v": np.zeros((1, 1, dim, tiles * 128), np.uint8), "qs": np.ones((1, 1, (nq + 63) // 64), np.float32),
            "ks": np.ones((1, 1, tiles), np.float32), "vs": np.ones((1, 1, dim), np.float32), "means": None,
            "qk_format": "fp8_block", "expcast": expcast, "block_values": False, "scale": 0.125}


@pytest.mark.parametrize("expcast", [False, True])
@pytest.mark.parametrize("nk", [1, 129, 257])
def test_fp8_zero_logits_tail_and_v_scale_known_answer(expcast, nk):
    # tests/test_fp8_qk.py:46-59: zero Q/K, V = 2 on the valid keys, vs = 3 -> 6 * weight.
    s = _fp8_payload(65, nk, expcast=expcast)
    s["v"][..., :nk] = o.e4m3_encode(np.float32(2.0))
    s["vs"][...] = 3.0
    weight = 1.0 if expcast else CONTROL_WEIGHT
    for affine in ((False, True) if expcast else (False,)):
        out = o.reference(s, affine=affine)
        np.testing.assert_allclose(out, 6 * weight, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("expcast", [False, True])
def test_fp8_sampling_keeps_block_scales(expcast):
    # tests/test_fp8_qk.py:24-43: rows sampled from 64-row blocks keep their own scale.
    gen = torch.Generator().manual_seed(2711)
    q = torch.randn(1, 2, 129, 64, generator=gen)
    k = torch.randn(1, 2, 257, 64, generator=gen)
    q[:, :, 64:128] *= 4
    k[:, :, 128:256] *= .125
    s = o.prepare_fp8(bits(q.to(torch.bfloat16)), bits(k.to(torch.bfloat16)),
                      bits(torch.randn(1, 2, 257, 64, generator=gen).to(torch.bfloat16)), expcast=expcast)
    ids = [0, 7, 63, 64, 65, 127, 128]
    for affine in ((False, True) if expcast else (False,)):
        full, fc = o.reference(s, return_codes=True, affine=affine)
        part, pc = o.reference(s, query_indices=ids, return_codes=True, affine=affine)
        np.testing.assert_array_equal(part, full[:, :, ids])
        np.testing.assert_array_equal(pc, fc[:, :, ids])


def test_fp8_control_path_is_a_softmax_of_the_block_dequantized_logits():
    # The scale of a score is qs[row // 64] * ks[key // 128] * sm (vc_reference.py:37-40):
    # the control output stays within the E4M3 bound of the float64 softmax of those logits,
    # and per-16-row or per-key-group scale indexing (the INT8 layout) would not.
    gen = torch.Generator().manual_seed(31)
    q = torch.randn(1, 1, 128, 64, generator=gen) * torch.tensor([1.0] * 64 + [4.0] * 64).view(1, 1, -1, 1)
    k = torch.randn(1, 1, 300, 64, generator=gen)
    k[:, :, 128:256] *= 0.125
    v = torch.randn(1, 1, 300, 64, generator=gen)
    s = o.prepare_fp8(*(bits(x.to(torch.bfloat16)) for x in (q, k, v)), expcast=False)
    out = o.reference(s)[0, 0].astype(np.float64)
    dq = o.e4m3_decode(s["q"][0, 0]).astype(np.float64) * np.repeat(s["qs"][0, 0], 64)[:128, None]
    dk = o.e4m3_decode(s["k"][0, 0]).astype(np.float64) * np.repeat(s["ks"][0, 0], 128)[:300, None]
    lg = dq @ dk.T * 0.125 * math.log2(math.e)
    w = np.exp2(lg - lg.max(-1, keepdims=True) + 8.807)
    dv = o.e4m3_decode(s["v"][0, 0, :, :300]).astype(np.float64) * s["vs"][0, 0, :, None]
    exact = (w @ dv.T) / w.sum(-1, keepdims=True)
    bound = ((2.0 ** -4 * w + 2.0 ** -10) @ np.abs(dv.T)) / w.sum(-1, keepdims=True)
    assert np.all(np.abs(out - exact) <= bound + 1e-4)
    # the check is sensitive to the scale indexing: K scales shifted by one tile break it
    dk2 = o.e4m3_decode(s["k"][0, 0]).astype(np.float64) * np.repeat(np.roll(s["ks"][0, 0], 1), 128)[:300, None]
    lg2 = dq @ dk2.T * 0.125 * math.log2(math.e)
    w2 = np.exp2(lg2 - lg2.max(-1, keepdims=True) + 8.807)
    wrong = (w2 @ dv.T) / w2.sum(-1, keepdims=True)
    assert np.mean(np.abs(wrong - exact) > bound) > 0.3


# ------------------------------------------------------------------ Hadamard Q/K rotation

def _explicit_hadamard(width):
    # Sylvester entries H[i,j] = (-1)**popcount(i & j) / sqrt(width), independent of the
    # butterfly (tests/test_paper_alignment.py:13-19).
    i = np.arange(width)
    pop = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    return (-1.0) ** pop / math.sqrt(width)


@pytest.mark.parametrize("dim", [1, 16, 37, 64, 128])
def test_hadamard_against_matrix_and_preserves_dot_products(dim):
    # tests/test_paper_alignment.py:22-29
    gen = torch.Generator().manual_seed(31)
    q, k = [torch.randn(2, 3, n, dim, generator=gen).numpy() for n in (7, 11)]
    width = 1 << (dim - 1).bit_length()
    hq, hk = o.hadamard(q), o.hadamard(k)
    expected = np.pad(q.astype(np.float64), [(0, 0)] * 3 + [(0, width - dim)]) @ _explicit_hadamard(width)
    np.testing.assert_allclose(hq, expected, atol=2e-6, rtol=2e-5)
    np.testing.assert_allclose(hq @ np.swapaxes(hk, -1, -2), q @ np.swapaxes(k, -1, -2), atol=2e-5, rtol=2e-5)
    # the rotation is an involution up to rounding: H(H(x)) = x
    np.testing.assert_allclose(o.hadamard(hq), np.pad(q, [(0, 0)] * 3 + [(0, width - dim)]), atol=3e-6)


def test_hadamard_butterfly_order_is_fixed():
    # Bit-exact values fix the stride order and the (left + right, left - right) pairing: a row
    # whose sums round differently under another stage order (large and small magnitudes).
    x = np.array([[1e8, 1.0, 3.0, -1e8, 0.5, 7.0, -2.0, 1e-3]], np.float32)
    want = x.astype(np.float32).copy()
    for s in (1, 2, 4):  # the reference's order (core.py:86-91)
        nxt = want.copy()
        for i in range(8):
            if not i & s:
                nxt[0, i] = np.float32(want[0, i] + want[0, i + s])
                nxt[0, i + s] = np.float32(want[0, i] - want[0, i + s])
        want = nxt
    want = want * np.float32(1 / math.sqrt(8))
    np.testing.assert_array_equal(o.hadamard(x), want)
    rev = x.astype(np.float32).copy()
    for s in (4, 2, 1):
        nxt = rev.copy()
        for i in range(8):
            if not i & s:
                nxt[0, i] = np.float32(rev[0, i] + rev[0, i + s])
                nxt[0, i + s] = np.float32(rev[0, i] - rev[0, i + s])
        rev = nxt
    assert not np.array_equal(rev * np.float32(1 / math.sqrt(8)), want)


@pytest.mark.parametrize("dim", [37, 64, 128])
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("k_smooth,rotate", [(False, False), (False, True), (True, False), (True, True)])
def test_preprocess_qk_matrix_oracle(dim, dtype, k_smooth, rotate):
    # tests/test_paper_alignment.py:124-150: K centred over all keys, then both rotated.
    gen = torch.Generator().manual_seed(14)
    q, k = [torch.randn(2, 2, n, dim, generator=gen) for n in (13, 35)]
    k += torch.linspace(-2, 2, dim)
    tdt = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[dtype]
    q, k = q.to(tdt), k.to(tdt)
    arg = (lambda x: x.numpy()) if dtype == "float32" else bits
    qo, ko = o.preprocess_qk(arg(q), arg(k), k_smooth=k_smooth, hadamard=rotate, dtype=dtype)
    eq, ek = q.double(), k.double()
    if k_smooth:
        ek = ek - ek.mean(-2, keepdim=True)
    if rotate:
        width = 1 << (dim - 1).bit_length()
        m = torch.from_numpy(_explicit_hadamard(width))
        eq = torch.nn.functional.pad(eq, (0, width - dim)) @ m
        ek = torch.nn.functional.pad(ek, (0, width - dim)) @ m
    np.testing.assert_allclose(qo, eq.numpy(), atol=3e-6, rtol=3e-5)
    np.testing.assert_allclose(ko, ek.numpy(), atol=3e-6, rtol=3e-5)


@pytest.mark.parametrize("D", [64, 128])
def test_rotated_int8_quantizers(D):
    # The rotated quantizers are the plain ones applied to the rotated rows: checked through
    # the per-thread invariants (|q8| <= 127, each group's maximum maps to +-127, the
    # dequantized rows within s/2 + ulp of the rotated rows) and the preserved dot products.
    q, k, _ = make_qkv(1, 2, 200, 300, D, torch.bfloat16, seed=8, kind="outlier")
    qb, kb = bits(q), bits(k)
    km = o.k_mean(kb)
    q8, qs = o.quant_q(qb, rotate=True)
    k8, ks = o.quant_k(kb, km, rotate=True)
    rq = o.hadamard(q.float().numpy())
    kmf = torch.from_numpy(np.ascontiguousarray(km).view(np.int16)).view(torch.bfloat16).float()
    kc = (k.float() - kmf.reshape(1, 2, 1, D)).to(torch.bfloat16).float().numpy()
    rk = o.hadamard(kc)
    rows = np.arange(200)
    sq = qs[:, :, (rows // 16) * 8 + rows % 8]
    deq = q8.astype(np.float64) * sq[..., None]
    assert np.all(np.abs(deq - rq) <= sq[..., None] / 2 * (1 + 1e-6) + 1e-6)
    assert np.abs(q8).max() == 127
    keys = np.arange(300)
    sk = ks[:, :, (keys // 128) * 4 + (keys % 8) // 2]
    dk = k8.astype(np.float64) * sk[..., None]
    assert np.all(np.abs(dk - rk) <= sk[..., None] / 2 * (1 + 1e-6) + 1e-6)
    # scores of the rotated payloads approximate the unrotated centred scores
    exact = q.double().numpy() @ np.swapaxes(kc.astype(np.float64), -1, -2)
    approx = deq @ np.swapaxes(dk, -1, -2)
    assert np.abs(approx - exact).max() <= 0.05 * np.abs(exact).max()
    # rotation changes the bytes (it is not silently skipped)
    assert not np.array_equal(q8, o.quant_q(qb)[0])


# ---- the control path's probability: correctly rounded binary32 exp2, then E4M3

def _round_f32(v):
    """Round a positive Fraction to the nearest binary32 (ties to even, subnormals included)."""
    from fractions import Fraction
    e = v.numerator.bit_length() - v.denominator.bit_length()
    while Fraction(2) ** e > v:
        e -= 1
    while Fraction(2) ** (e + 1) <= v:
        e += 1
    q = max(e - 23, -149)
    scaled = v / Fraction(2) ** q
    n = scaled.numerator // scaled.denominator
    r = scaled - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return np.float32(float(Fraction(n) * Fraction(2) ** q))


def _exp2_decimal(x):
    """binary32 exp2(x) from a 60-digit decimal evaluation, rounded once."""
    from decimal import Decimal, localcontext
    from fractions import Fraction
    with localcontext() as ctx:
        ctx.prec = 60
        d = (Decimal(float(x)) * Decimal(2).ln()).exp()
    return _round_f32(Fraction(d))


def test_exp2_rn_is_correctly_rounded():
    # integers give exact powers of two (subnormal results included)
    for k in range(-149, 128):
        assert o.exp2_rn(k) == 2.0 ** k, k
    assert o.exp2_rn(-150) == 0.0  # 2^-150 is the tie between 0 and 2^-149: even is 0
    assert np.isinf(o.exp2_rn(128.0)) and o.exp2_rn(-np.inf) == 0.0
    rng = np.random.default_rng(5)
    xs = list(rng.uniform(-12, 9, 1500).astype(np.float32)) + list(rng.uniform(-1e-3, 1e-3, 200).astype(np.float32))
    # inputs whose exp2 lies next to an E4M3 rounding midpoint (where the control path's byte
    # depends on the binary32 rounding): x0 = RN(log2 M) and its neighbours
    codes = [c for c in range(1, 126)]
    vals = [float(o.e4m3_decode(np.array([c], np.uint8))[0]) for c in codes + [126]]
    for lo, hi in zip(vals[:-1], vals[1:]):
        x0 = np.float32(np.log2((lo + hi) / 2))
        xs += list((np.array([x0]).view(np.int32) + np.arange(-12, 13)).astype(np.int32).view(np.float32))
    for x in xs:
        assert o.exp2_rn(x) == _exp2_decimal(x), float(x)


def test_fp8_exp2_codes_known_answers():
    # p = exp2(x): 2^0 = 1 -> 0x38; 2^-1 -> 0x30; the offset maximum 2^8.807 ~ 447.9 -> 448 (0x7E);
    # 2^-10 is the tie between 0 and the smallest subnormal 2^-9 (even: 0); just above it: 2^-9
    x = np.array([0.0, -1.0, 8.807, -10.0, np.nextafter(np.float32(-10.0), np.float32(0)), -np.inf, -20.0],
                 np.float32)
    np.testing.assert_array_equal(o.fp8_exp2_codes(x), [0x38, 0x30, 0x7E, 0, 1, 0, 0])
    # the sweep form equals the array form
    first = int(np.float32(-3.0).view(np.uint32))
    xs = (np.uint32(first) + np.arange(4096, dtype=np.uint32)).view(np.float32)
    np.testing.assert_array_equal(o.fp8_exp2_sweep(first, 4096), o.fp8_exp2_codes(xs))
    np.testing.assert_array_equal(o.fp8_exp2_codes(xs), o.e4m3_encode([o.exp2_rn(v) for v in xs]))
