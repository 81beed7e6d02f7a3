"""GPU parity of libvcx (through its C ABI) against the CPU oracle.

Bit-exact: ExpCast codes, conversions, INT8 Q/K payloads and scales, K mean,
E4M3 V payloads (logical order), V scales and fp16 means, grouping labels /
permutation / centers, and the E4M3 P bytes produced inside the fused kernel.
Tolerance (written in helpers.output_bound): the fp16/bf16 attention output vs
the oracle's decoded-payload path, plus cosine >= 0.9999.
"""
import numpy as np
import pytest
import torch

import vcx
from helpers import (FOLD_CODE_FOLDED, FOLD_CODE_UNFUSED, bits, cosine, dtype_name, folded_encode_payload,
                     logical_to_storage, make_qkv, output_bound, storage_to_logical)
from oracle import vc_oracle as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _print_case(*args):
    print("case:", *args, flush=True)


def test_device_is_gfx950_and_library_loaded():
    assert torch.cuda.is_available()
    arch = torch.cuda.get_device_properties(DEV).gcnArchName
    assert arch.startswith("gfx950"), arch
    assert vcx.abi_version() == vcx.ABI_VERSION
    tok = vcx.value_token()
    assert sorted(tok) == list(range(128))


def test_clock_probe_reads_a_plausible_engine_clock():
    # 2 ms of real time: the engine counter must run between 0.5 and 3 GHz, and a window
    # twice as long must read about twice the real-time ticks.
    short, long_ = vcx.clock_probe(2000, DEV), vcx.clock_probe(4000, DEV)
    ghz = short.ghz()
    assert 0.5 < ghz < 3.0, ghz
    assert 0.5 < long_.ghz() < 3.0
    assert short.wall_khz > 0
    assert all(0.5 < g < 3.0 for g in short.ghz_per_block())
    ratio = int(long_.ticks[1]) / int(short.ticks[1])
    assert 1.9 < ratio < 2.1, ratio


# ------------------------------------------------------------------ scalar maps

def test_expcast_codes_sweep_bit_exact():
    # scripts/validate_sage_vc.py:22-24 sweep, plus every code boundary +- 8 ulps.
    xs = [np.linspace(-15, 1, 65537, dtype=np.float32), np.array([-np.inf, -20.0, 0.0, np.nan, 3.0], np.float32)]
    A, B = np.float32(11.541560173034668), np.float32(119.6500015258789)
    for c in range(0, 121):
        x0 = np.float32((c + 0.5 - np.float64(B)) / np.float64(A))
        xs.append((x0.view(np.int32) + np.arange(-8, 9)).astype(np.int32).view(np.float32))
    x = np.concatenate(xs).astype(np.float32)
    _print_case("expcast sweep", x.size)
    got = vcx.expcast_codes(torch.from_numpy(x).to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, o.expcast_codes(x))


def test_conversion_instructions_bit_exact():
    rng = np.random.default_rng(5)
    parts = [np.array([-np.inf, np.inf, 0.0, -0.0, 1e-30, -1e-30, 1e-45], np.float32)]
    for k in range(-2, 257):  # every half-integer +- 64 ulps (cvt_pk_u8 rounding)
        h = np.float32(k + 0.5)
        parts.append((h.view(np.int32) + np.arange(-64, 65)).astype(np.int32).view(np.float32))
    dec = o.e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    for a, b in zip(dec[:-1], dec[1:]):  # every E4M3 midpoint +- 64 ulps, both signs
        m = np.float32((a + b) / 2)
        s = (m.view(np.int32) + np.arange(-64, 65)).astype(np.int32).view(np.float32)
        parts += [s, -s]
    parts.append((rng.standard_normal(1 << 20) * 200).astype(np.float32))
    parts.append(np.ldexp(rng.random(1 << 20), rng.integers(-20, 10, 1 << 20)).astype(np.float32))
    x = np.concatenate(parts)
    _print_case("conversion probe", x.size)
    u8, f8 = vcx.convert_probe(torch.from_numpy(x).to(DEV))
    np.testing.assert_array_equal(u8.cpu().numpy(), o.cvt_u8(x))
    np.testing.assert_array_equal(f8.cpu().numpy(), o.e4m3_encode(np.clip(x, -448, 448)))


# ------------------------------------------------------------------ preprocessing

SHAPES = [  # B, H, Nq, Nk, D, dtype
    (1, 2, 2048, 2048, 128, torch.bfloat16),
    (1, 1, 1, 1, 128, torch.bfloat16),
    (2, 3, 65, 129, 64, torch.float16),
    (1, 2, 257, 385, 128, torch.float16),
    (1, 1, 63, 127, 64, torch.bfloat16),
    (1, 1, 300, 4097, 128, torch.bfloat16),
]


def _ids(shape):
    return "B%dH%dq%dk%dD%d%s" % (*shape[:5], "bf16" if shape[5] == torch.bfloat16 else "f16")


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
@pytest.mark.parametrize("kind", ["normal", "outlier"])
def test_prepare_qk_bit_exact(shape, kind):
    B, H, Nq, Nk, D, dt = shape
    _print_case("prepare_qk", _ids(shape), kind)
    q, k, v = make_qkv(B, H, Nq, Nk, D, dt, seed=1, kind=kind)
    q8, qs, k8, ks, km = vcx.prepare_qk(q.to(DEV), k.to(DEV))
    name = dtype_name(dt)
    ekm = o.k_mean(bits(k), None, name)
    eq8, eqs = o.quant_q(bits(q), name)
    ek8, eks = o.quant_k(bits(k), ekm, None, name)
    np.testing.assert_array_equal(km.view(torch.int16).cpu().numpy().view(np.uint16).reshape(B, H, D), ekm)
    np.testing.assert_array_equal(q8.cpu().numpy(), eq8)
    np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint32), eqs.view(np.uint32))
    np.testing.assert_array_equal(k8.cpu().numpy(), ek8)
    np.testing.assert_array_equal(ks.cpu().numpy().view(np.uint32), eks.view(np.uint32))


def test_prepare_qk_strided_nhd_and_permutation():
    B, H, N, D = 1, 3, 333, 128
    q, k, v = make_qkv(B, H, N, N, D, torch.bfloat16, seed=3)
    g = torch.Generator().manual_seed(4)
    perm = torch.stack([torch.randperm(N, generator=g) for _ in range(B * H)]).view(B, H, N)
    qn, kn = (x.transpose(1, 2).contiguous().to(DEV) for x in (q, k))  # NHD storage
    q8, qs, k8, ks, km = vcx.prepare_qk(qn.transpose(1, 2), kn.transpose(1, 2), perm.to(DEV))
    ekm = o.k_mean(bits(k), perm.numpy())
    ek8, eks = o.quant_k(bits(k), ekm, perm.numpy())
    eq8, eqs = o.quant_q(bits(q))
    np.testing.assert_array_equal(q8.cpu().numpy(), eq8)
    np.testing.assert_array_equal(k8.cpu().numpy(), ek8)
    np.testing.assert_array_equal(ks.cpu().numpy().view(np.uint32), eks.view(np.uint32))
    np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint32), eqs.view(np.uint32))


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
@pytest.mark.parametrize("mode", ["channel_fp8", "smooth_channel", "smooth_block"])
def test_prepare_v_bit_exact(shape, mode):
    B, H, Nq, Nk, D, dt = shape
    _print_case("prepare_v", _ids(shape), mode)
    _, _, v = make_qkv(B, H, Nq, Nk, D, dt, seed=2, kind="outlier")
    if Nk > 3:
        v[0, 0, :, 3] = 0  # zero channel
    name = dtype_name(dt)
    smooth = mode != "channel_fp8"
    channel = mode != "smooth_block"
    v8, vs, means = vcx.prepare_v(v.to(DEV), None, smooth=smooth, channel_scale=channel)
    tok = vcx.value_token()
    got = storage_to_logical(v8, tok)
    if smooth:
        ev8, evs, emeans = o.prepare_values(bits(v), None, channel, name)
        np.testing.assert_array_equal(means.view(torch.int16).cpu().numpy().view(np.uint16), emeans)
    else:
        ev8, evs = o.per_channel_fp8(bits(v), None, name)
    np.testing.assert_array_equal(got, ev8)
    np.testing.assert_array_equal(vs.cpu().numpy().view(np.uint32), evs.view(np.uint32))


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n,clusters,iterations", [(1, 8, 2), (7, 8, 1), (127, 3, 3), (128, 1, 2), (129, 8, 2),
                                                   (2049, 8, 2), (5000, 8, 3)])
def test_grouping_bit_exact(dim, dtype, n, clusters, iterations):
    _print_case("grouping", dim, dtype, n, clusters, iterations)
    torch.manual_seed(211 + n)
    v = torch.randn(2, 2, n, dim).to(dtype)
    perm, labels, centers = vcx.group_values(v.to(DEV), clusters, iterations, debug=True)
    eperm, elabels, ecenters = o.group_values(bits(v), clusters, iterations, dtype_name(dtype))
    np.testing.assert_array_equal(labels.cpu().numpy(), elabels)
    np.testing.assert_array_equal(centers.cpu().numpy().view(np.uint32), ecenters.view(np.uint32))
    np.testing.assert_array_equal(perm.cpu().numpy(), eperm)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("clusters", [8, 16])
@pytest.mark.parametrize("bad", ["nan", "inf"])
def test_grouping_non_finite_values_follow_the_oracle(dim, clusters, bad):
    # A non-finite V value gives NaN / infinite distances; the kernel's binary32 pre-pass must
    # leave such tokens to the fp64 chains (ties and NaN compares resolve to the lowest id), so
    # labels, centers and the permutation equal the oracle's. Reference assignment rule:
    # clustering.cu:32-137 (first minimum wins).
    _print_case("grouping non-finite", dim, clusters, bad)
    g = torch.Generator().manual_seed(5 + dim + clusters)
    v = torch.randn(1, 2, 700, dim, generator=g)
    v[0, 0, 123, 7] = float(bad)
    v[0, 1, 0, 3] = -float(bad) if bad == "inf" else float(bad)  # an initial center of head 1
    v = v.to(torch.bfloat16)
    perm, labels, centers = vcx.group_values(v.to(DEV), clusters, 2, debug=True)
    eperm, elabels, ecenters = o.group_values(bits(v), clusters, 2, "bfloat16")
    np.testing.assert_array_equal(labels.cpu().numpy(), elabels)
    np.testing.assert_array_equal(perm.cpu().numpy(), eperm)
    np.testing.assert_array_equal(centers.cpu().numpy(), ecenters)  # NaN == NaN here


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("offset", [0.0, 40.0, 3.0e4])
def test_grouping_offset_values_follow_the_oracle(dim, offset):
    # V = offset + N(0, 1) in bf16: with a large offset |x|^2 + |c|^2 dwarfs |x - c|^2, so the
    # kernel's dot-product pre-pass (x.c on the MFMA) cannot settle many tokens and leaves
    # them to the binary32 and fp64 chains, inside waves where others are settled; bf16's
    # coarse steps at the offset also make exact distance ties. Labels, centers and the
    # permutation must still be the oracle's.
    _print_case("grouping offset", dim, offset)
    g = torch.Generator().manual_seed(17 + dim)
    v = (offset + torch.randn(1, 2, 3000, dim, generator=g)).to(torch.bfloat16)
    perm, labels, centers = vcx.group_values(v.to(DEV), 8, 3, debug=True)
    eperm, elabels, ecenters = o.group_values(bits(v), 8, 3, "bfloat16")
    np.testing.assert_array_equal(labels.cpu().numpy(), elabels)
    np.testing.assert_array_equal(centers.cpu().numpy().view(np.uint32), ecenters.view(np.uint32))
    np.testing.assert_array_equal(perm.cpu().numpy(), eperm)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_grouping_rows_not_16_byte_aligned(dim, dtype):
    # a token stride of dim + 2 elements leaves rows 4-byte aligned only: the tile is staged in
    # 4-byte pieces, one tile per block (the bf16 pre-pass without the next tile's loads in
    # flight); labels, centers, next centers and the permutation are still the oracle's.
    _print_case("grouping unaligned rows", dim, dtype)
    g = torch.Generator().manual_seed(31 + dim)
    v = torch.randn(1, 2, 1500, dim, generator=g).to(dtype)
    wide = torch.zeros(1, 2, 1500, dim + 2, dtype=dtype)
    wide[..., :dim] = v
    dv = wide.to(DEV)[..., :dim]
    assert dv.stride(2) % 8 != 0
    perm, labels, centers, nxt = vcx.group_values(dv, 8, 2, debug=True, return_centers=True)
    eperm, elabels, ecenters, enext = o.group_values(bits(v), 8, 2, dtype_name(dtype), return_next=True)
    np.testing.assert_array_equal(labels.cpu().numpy(), elabels)
    np.testing.assert_array_equal(centers.cpu().numpy().view(np.uint32), ecenters.view(np.uint32))
    np.testing.assert_array_equal(nxt.cpu().numpy().view(np.uint32), enext.view(np.uint32))
    np.testing.assert_array_equal(perm.cpu().numpy(), eperm)


@pytest.mark.parametrize("dim", [64, 128])
def test_grouping_zero_padding_rows(dim):
    # Zero rows at the end of each head (padding): four initial centers are the same zero row,
    # so most tokens tie between them exactly, in every wave (each lane's own binary32 and fp64
    # chains). Labels, centers, next centers and the permutation are the oracle's.
    _print_case("grouping zero padding", dim)
    g = torch.Generator().manual_seed(43 + dim)
    v = torch.randn(1, 2, 1400, dim, generator=g)
    v[:, :, 700:] = 0.0
    v = v.to(torch.bfloat16)
    perm, labels, centers, nxt = vcx.group_values(v.to(DEV), 8, 2, debug=True, return_centers=True)
    eperm, elabels, ecenters, enext = o.group_values(bits(v), 8, 2, "bfloat16", return_next=True)
    np.testing.assert_array_equal(labels.cpu().numpy(), elabels)
    np.testing.assert_array_equal(centers.cpu().numpy().view(np.uint32), ecenters.view(np.uint32))
    np.testing.assert_array_equal(nxt.cpu().numpy().view(np.uint32), enext.view(np.uint32))
    np.testing.assert_array_equal(perm.cpu().numpy(), eperm)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("every", [16, 64])
def test_grouping_few_near_ties_per_wave(dim, every):
    # The near-tie tokens below, but only every 16th (4 per 64-token wave) or 64th stays on
    # the bisector; the others move to one side (settled by the bf16 pre-pass). A wave's few
    # open tokens go through the wave-wide binary32 stage one at a time and, exact and near
    # ties, through the fp64 chains 8 rows at a time; labels and permutation are the oracle's.
    _print_case("grouping few near ties", dim, every)
    v = _near_tie_values(dim, torch.bfloat16).float()
    n = v.shape[2]
    t = torch.arange(n)
    side = (t % every != 5) & (t > 0) & (t < n - 1)
    v[0, :, side, 0] = torch.where(t[side] % 2 == 0, 0.75, -0.75)
    v = v.to(torch.bfloat16)
    perm, labels, centers = vcx.group_values(v.to(DEV), 2, 1, debug=True)
    eperm, elabels, ecenters = o.group_values(bits(v), 2, 1, "bfloat16")
    np.testing.assert_array_equal(labels.cpu().numpy(), elabels)
    np.testing.assert_array_equal(perm.cpu().numpy(), eperm)
    tie = (t.numpy() % every == 5) & (t.numpy() % 3 == 1) & (t.numpy() % 7 != 0)
    assert tie.any() and np.all(elabels[..., tie] == 0)


def _near_tie_values(dim, dtype, n=1024, seed=0):
    """[1,2,n,dim] V whose tokens sit at or near the bisector of the two initial centers
    (V[0] = -e_0 + w, V[n-1] = +e_0 + w, with the same random tail w in the other channels):
    token t has channel 0 = s_t * 2^-k (k = 9..24, s_t in {-1, 0, +1}) and the tail w plus
    small noise on a few tokens. Its two distances differ by 4 * channel 0, i.e. down to a
    relative 2^-24 / (1 + |w|^2), far inside the binary32 error of the distance sums, so
    the kernel's binary32 pass must leave these tokens to the fp64 chains; s_t = 0 gives exact
    ties (lowest id)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(2, dim, generator=g).to(dtype).float()
    w[:, 0] = 0
    v = w[:, None, :].repeat(1, n, 1)
    t = torch.arange(n)
    k = 9 + t % 16
    sgn = (t % 3 - 1).float()
    v[:, :, 0] = sgn[None, :] * torch.pow(2.0, -k.float())[None, :]
    noisy = t % 7 == 0
    v[:, noisy, 1:] += 0.5 * torch.randn(2, int(noisy.sum()), dim - 1, generator=g)
    v[:, 0, :] = w
    v[:, 0, 0] = -1.0
    v[:, n - 1, :] = w
    v[:, n - 1, 0] = 1.0
    return v[None].to(dtype)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("legacy", [False, True])
def test_grouping_near_ties_take_the_fp64_chains(dim, dtype, legacy):
    # Labels are the fp64 argmin (ties to the lowest id); a binary32 pass decides only when
    # its order is certain. Tokens on and next to the bisector of the two centers must get
    # the oracle's labels exactly, through both schedules.
    _print_case("grouping near ties", dim, dtype, legacy)
    v = _near_tie_values(dim, dtype)
    perm, labels, centers = vcx.group_values(v.to(DEV), 2, 1, debug=True, legacy=legacy)
    eperm, elabels, ecenters = o.group_values(bits(v), 2, 1, dtype_name(dtype))
    np.testing.assert_array_equal(labels.cpu().numpy(), elabels)
    np.testing.assert_array_equal(perm.cpu().numpy(), eperm)
    # both labels occur, and exact ties went to cluster 0
    assert 0 < elabels.mean() < 1
    n = v.shape[2]
    tie = (np.arange(n) % 3 == 1) & (np.arange(n) % 7 != 0) & (np.arange(n) > 0) & (np.arange(n) < n - 1)
    assert np.all(elabels[..., tie] == 0)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("n,clusters,iterations", [(2049, 16, 2), (1000, 64, 3), (600, 256, 2), (100, 256, 2),
                                                   (129, 9, 2), (37741, 32, 2)])
def test_grouping_many_clusters_bit_exact(dim, n, clusters, iterations):
    # 9..256 effective clusters take the general schedule (the reference's legacy range,
    # pybind.cpp:6-44); labels, perm, both center sets bit-exact against the oracle.
    _print_case("grouping many", dim, n, clusters, iterations)
    torch.manual_seed(401 + n + clusters)
    heads = 1 if n > 10000 else 2
    v = torch.randn(1, heads, n, dim).to(torch.bfloat16)
    perm, labels, centers, nxt = vcx.group_values(v.to(DEV), clusters, iterations, debug=True, return_centers=True)
    eperm, elabels, ecenters, enext = o.group_values(bits(v), clusters, iterations, return_next=True)
    np.testing.assert_array_equal(labels.cpu().numpy(), elabels)
    np.testing.assert_array_equal(centers.cpu().numpy().view(np.uint32), ecenters.view(np.uint32))
    np.testing.assert_array_equal(nxt.cpu().numpy().view(np.uint32), enext.view(np.uint32))
    np.testing.assert_array_equal(perm.cpu().numpy(), eperm)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n,clusters,iterations", [(1, 8, 2), (127, 3, 3), (2049, 8, 2), (5000, 8, 3)])
def test_grouping_general_schedule_equals_fused(dtype, n, clusters, iterations):
    # grouping_mode="legacy" runs the general schedule for every count; at <= 8 clusters it
    # must give the fused schedule's bits exactly (and the oracle's).
    _print_case("grouping legacy == fused", dtype, n, clusters, iterations)
    torch.manual_seed(5 + n)
    v = torch.randn(2, 2, n, 128).to(dtype).to(DEV)
    fused = vcx.group_values(v, clusters, iterations, debug=True, return_centers=True)
    general = vcx.group_values(v, clusters, iterations, debug=True, return_centers=True, legacy=True)
    for a, b in zip(fused, general):
        assert torch.equal(a, b)
    eperm, elabels, ecenters, enext = o.group_values(bits(v.cpu()), clusters, iterations, dtype_name(dtype),
                                                     return_next=True)
    np.testing.assert_array_equal(general[0].cpu().numpy(), eperm)
    np.testing.assert_array_equal(general[3].cpu().numpy().view(np.uint32), enext.view(np.uint32))


@pytest.mark.parametrize("legacy", [False, True])
@pytest.mark.parametrize("clusters", [8, 16])
def test_grouping_warm_start_bit_exact(legacy, clusters):
    # a cached layout's refresh starts from the previous call's next centers
    # (src/vc_attention/core.py:216-221); strided NHD input on a side stream.
    _print_case("grouping warm start", legacy, clusters)
    torch.manual_seed(9)
    v0 = torch.randn(1, 3, 700, 128).to(torch.bfloat16)
    v1 = (v0.float() + 0.3 * torch.randn(1, 3, 700, 128)).to(torch.bfloat16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        d1 = v1.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)  # NHD storage, HND view
        _, cached = vcx.group_values(v0.to(DEV), clusters, 2, legacy=legacy, return_centers=True)
        perm, labels, centers, nxt = vcx.group_values(d1, clusters, 2, debug=True, legacy=legacy, centers=cached,
                                                      return_centers=True)
    side.synchronize()
    _, _, _, ecached = o.group_values(bits(v0), clusters, 2, return_next=True)
    np.testing.assert_array_equal(cached.cpu().numpy().view(np.uint32), ecached.view(np.uint32))
    eperm, elabels, ecenters, enext = o.group_values(bits(v1), clusters, 2, centers_in=ecached, return_next=True)
    np.testing.assert_array_equal(labels.cpu().numpy(), elabels)
    np.testing.assert_array_equal(centers.cpu().numpy().view(np.uint32), ecenters.view(np.uint32))
    np.testing.assert_array_equal(nxt.cpu().numpy().view(np.uint32), enext.view(np.uint32))
    np.testing.assert_array_equal(perm.cpu().numpy(), eperm)


def test_grouping_known_answers():
    x = torch.tensor([2, 0, 1, 2, 1, 0], dtype=torch.float32)
    v = x.view(1, 1, 6, 1).expand(2, 2, 6, 64).contiguous().to(torch.bfloat16).to(DEV)
    perm = vcx.group_values(v, 3, 2)
    for row in perm.cpu().reshape(-1, 6):
        assert row.tolist() == [0, 3, 2, 4, 1, 5]
    v = torch.full((2, 3, 257, 128), 2.0, dtype=torch.bfloat16, device=DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        perm, labels, centers = vcx.group_values(v, 8, 3, debug=True)
        total = labels.sum()
    stream.synchronize()
    assert total.item() == 0
    assert torch.equal(perm.cpu(), torch.arange(257).expand(2, 3, 257))
    assert (centers == 2).all().item()


# ------------------------------------------------------------------ fused attention

def _to_dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(DEV)


def _oracle_state(q, k, v, smooth, dt):
    return o.prepare(bits(q), bits(k), bits(v), v_smooth=smooth, dtype=dtype_name(dt))


ATTN = [  # B, H, Nq, Nk, D, dtype, smooth
    (1, 2, 2048, 2048, 128, torch.bfloat16, False),
    (1, 2, 2048, 2048, 128, torch.bfloat16, True),
    (1, 1, 1, 1, 128, torch.bfloat16, False),
    (2, 3, 65, 129, 64, torch.float16, True),
    (1, 2, 257, 385, 128, torch.float16, False),
    (1, 1, 63, 127, 64, torch.bfloat16, False),
    (1, 1, 129, 513, 64, torch.bfloat16, True),
    (1, 1, 200, 4097, 128, torch.bfloat16, True),
]


@pytest.mark.parametrize("case", ATTN, ids=lambda c: _ids(c[:6]) + ("_smooth" if c[6] else ""))
def test_attention_p_bytes_bit_exact_and_output_tolerance(case):
    B, H, Nq, Nk, D, dt, smooth = case
    _print_case("attention", case)
    q, k, v = make_qkv(B, H, Nq, Nk, D, dt, seed=7, kind="outlier" if smooth else "normal")
    st = _oracle_state(q, k, v, smooth, dt)
    tok = vcx.value_token()
    # Feed the kernel the oracle's payloads (storage order) so the kernel is tested on its own.
    to = _to_dev
    v8 = to(logical_to_storage(st["v"], tok)).view(torch.float8_e4m3fn)
    means = to(st["means"]).view(torch.float16) if smooth else None
    rows = (0, Nq)
    out, pd = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]), means,
                          True, smooth, st["output_type"], st["scale"], p_rows=rows)
    eout, ecodes = o.reference(st, return_codes=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound), float((err - bound).max())
    assert cosine(got, eout) >= 0.9999
    # the production (non-dump) kernel gives the same output bits
    out2 = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]), means,
                       True, smooth, st["output_type"], st["scale"])
    assert torch.equal(out2, out)


def test_uniform_attention_three_unequal_blocks_known_answer():
    # scripts/validate_sage_vc.py:479-492: q = k = 0, three unequal V blocks; output = mean of V.
    from sageattention_local import sageattn_vc
    for dtype in (torch.float16, torch.bfloat16):
        q = torch.zeros(1, 2, 65, 128, device=DEV, dtype=dtype)
        k = torch.zeros(1, 2, 257, 128, device=DEV, dtype=dtype)
        channels = torch.linspace(-2, 2, 128, device=DEV)
        v = torch.empty_like(k)
        v[:, :, :128] = channels
        v[:, :, 128:256] = channels * 2 + 3
        v[:, :, 256:] = channels * 0.25 - 6
        expected = v.float().mean(2, keepdim=True).expand_as(q).to(dtype)
        # With smoothing every block is its own mean: residual bytes are zero and the
        # mean restoration alone must give the exact average (the reference's check).
        out = sageattn_vc(q, k, v, expcast=True, v_smooth=True)
        torch.testing.assert_close(out, expected, rtol=0.004, atol=0.004)
        # Without smoothing the weights are still uniform: the output is the mean of
        # the DECODED FP8 payload times the channel scale.
        state_v8, vs, _ = vcx.prepare_v(v)
        dec = torch.from_numpy(o.e4m3_decode(storage_to_logical(state_v8, vcx.value_token())[..., :257]))
        expected_fp8 = (dec.double().mean(-1) * vs.cpu().double()).unsqueeze(2).expand(1, 2, 65, 128)
        out = sageattn_vc(q, k, v, expcast=True, v_smooth=False)
        torch.testing.assert_close(out.double().cpu(), expected_fp8, rtol=0.004, atol=0.004)


def test_sageattn_vc_end_to_end_config1_payloads_and_output():
    # Config 1 of the benchmark: BNSD [1,2,2048,128] bf16, smoothing off and on.
    from sageattention_local import prepare, forward_prepared, sageattn_vc
    q, k, v = make_qkv(1, 2, 2048, 2048, 128, torch.bfloat16, seed=0)
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    tok = vcx.value_token()
    for smooth in (False, True):
        _print_case("end-to-end config1", smooth)
        st = prepare(qd, kd, vd, v_smooth=smooth)
        ost = _oracle_state(q, k, v, smooth, torch.bfloat16)
        for key in ("q", "k", "qs", "ks"):
            np.testing.assert_array_equal(st[key].cpu().numpy(), ost[key])
        np.testing.assert_array_equal(storage_to_logical(st["v"], tok), ost["v"])
        np.testing.assert_array_equal(st["vs"].cpu().numpy(), ost["vs"])
        if smooth:
            np.testing.assert_array_equal(st["permutation"].cpu().numpy(), ost["permutation"])
            np.testing.assert_array_equal(st["means"].view(torch.int16).cpu().numpy().view(np.uint16), ost["means"])
        out = forward_prepared(st).float().cpu().numpy()
        # the default kernel mode folds the ExpCast encode when there are no block values
        eout = o.reference(ost, affine=not smooth)
        err, bound = output_bound(out, eout)
        assert np.all(err <= bound)
        assert cosine(out, eout) >= 0.9999
        full = sageattn_vc(qd, kd, vd, v_smooth=smooth)
        assert torch.equal(full.float().cpu(), torch.from_numpy(out))


def test_hnd_and_nhd_layouts_exact():
    # scripts/validate_sage_vc.py:493-498
    from sageattention_local import sageattn_vc
    q, k, v = (x.to(DEV) for x in make_qkv(1, 2, 257, 300, 128, torch.bfloat16, seed=338))
    for smooth in (False, True):
        hnd = sageattn_vc(q, k, v, v_smooth=smooth)
        nhd = sageattn_vc(*(x.transpose(1, 2).contiguous() for x in (q, k, v)), tensor_layout="NHD", v_smooth=smooth)
        assert torch.equal(hnd, nhd.transpose(1, 2))


def test_full_length_prep_exact_and_sampled_p_bytes():
    # The main shape's sequence length (37741) with 2 heads: every payload byte,
    # and P bytes of a sampled row range, against the oracle.
    B, H, N, D = 1, 2, 37741, 128
    q, k, v = make_qkv(B, H, N, N, D, torch.bfloat16, seed=0)
    _print_case("full-length", N)
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    q8, qs, k8, ks, km = vcx.prepare_qk(qd, kd)
    v8, vs, _ = vcx.prepare_v(vd)
    st = _oracle_state(q, k, v, False, torch.bfloat16)
    np.testing.assert_array_equal(q8.cpu().numpy(), st["q"])
    np.testing.assert_array_equal(k8.cpu().numpy(), st["k"])
    np.testing.assert_array_equal(qs.cpu().numpy(), st["qs"])
    np.testing.assert_array_equal(ks.cpu().numpy(), st["ks"])
    np.testing.assert_array_equal(storage_to_logical(v8, vcx.value_token()), st["v"])
    np.testing.assert_array_equal(vs.cpu().numpy(), st["vs"])
    r0, r1 = 18800, 18816
    out, pd = vcx.forward(q8, k8, v8, qs, ks, vs, None, True, False, 1, D ** -0.5, p_rows=(r0, r1))
    eout, ecodes = o.reference(st, query_indices=np.arange(r0, r1), return_codes=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out[:, :, r0:r1].float().cpu().numpy()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound)
    assert cosine(got, eout) >= 0.9999


def test_block_list_writes_every_row_and_halves_match_the_oracle():
    # [1,2,37741,128] makes 590 128-row blocks. Each XCD takes a contiguous range of them, and
    # the last blocks of every range run as two 64-row blocks. On a 256-CU MI355X the chosen
    # split makes rows 8192..9471 of both heads 64-row blocks (the end of the first and of the
    # fifth XCD's range). Every output row must be written, and those rows must carry the
    # oracle's P bytes (folded encode) and output.
    B, H, N, D = 1, 2, 37741, 128
    q, k, v = make_qkv(B, H, N, N, D, torch.bfloat16, seed=3)
    _print_case("block list", N)
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    q8, qs, k8, ks, _ = vcx.prepare_qk(qd, kd)
    v8, vs, _ = vcx.prepare_v(vd)
    out = torch.full((B, H, N, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    vcx.forward(q8, k8, v8, qs, ks, vs, None, True, False, 1, D ** -0.5, affine=True, out=out)
    assert bool(torch.isfinite(out).all())
    st = _oracle_state(q, k, v, False, torch.bfloat16)
    r0, r1 = 8192, 9472
    out2, pd = vcx.forward(q8, k8, v8, qs, ks, vs, None, True, False, 1, D ** -0.5, affine=True, p_rows=(r0, r1))
    assert torch.equal(out2, out)
    eout, ecodes = o.reference(st, query_indices=np.arange(r0, r1), return_codes=True, affine=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out[:, :, r0:r1].float().cpu().numpy()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound)
    assert cosine(got, eout) >= 0.9999


@pytest.mark.parametrize("nk", [2, 129, 300])
def test_last_tile_rounding_order_known_answer_on_gpu(nk):
    # The fused kernel's P bytes on the rounding-order payload: byte 96 when the pair of
    # keys is in the last tile, 97 when it is in an earlier tile (oracle known answer).
    from helpers import ORDER_CODE_LAST, ORDER_CODE_OTHER, rounding_order_payload
    _print_case("rounding order", nk)
    st = rounding_order_payload(nk)
    to = _to_dev
    v8 = to(st["v"]).view(torch.float8_e4m3fn)
    _, pd = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]), None,
                        True, False, 1, st["scale"], p_rows=(0, 1))
    codes = pd.cpu().numpy()
    assert codes[0, 0, 0, 0] == 120
    assert codes[0, 0, 0, 1] == (ORDER_CODE_LAST if nk <= 128 else ORDER_CODE_OTHER)
    assert np.all(codes[0, 0, 0, 2:] == 0)


FULL = [  # name, B, H, N, D, kind: the BASELINE smoothing configurations in full
    ("smooth", 1, 28, 37741, 128, "outlier"),
    ("d64", 1, 40, 32760, 64, "normal"),
    ("long", 1, 28, 75482, 128, "student"),
]


@pytest.mark.timeout(900)  # the long case draws 2 x 270M Student-t values on one CPU core (~1 min)
@pytest.mark.parametrize("case", FULL, ids=lambda c: c[0])
def test_full_length_baseline_configs_all_heads(case):
    # The BASELINE smoothing shapes in full (all 28 / 40 heads, full sequence length) on the
    # very bytes bench.py times (bench.make_inputs: CPU torch.Generator seed 0, numpy PCG64
    # Student-t for "long"): the permutation, every Q8/K8/V8 byte, every scale and fp16 mean
    # of every head; then P bytes and output of sampled rows (first, middle, ragged end) in
    # every head.
    from bench import make_inputs
    from sageattention_local import forward_prepared, prepare
    name, B, H, N, D, kind = case
    _print_case("full config, all heads, bench inputs", name, (B, H, N, D))
    q, k, v = make_inputs(B, H, N, D, kind)
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    st = prepare(qd, kd, vd, v_smooth=True)
    ost = _oracle_state(q, k, v, True, torch.bfloat16)
    np.testing.assert_array_equal(st["permutation"].cpu().numpy(), ost["permutation"])
    for key in ("q", "k", "qs", "ks", "vs"):
        np.testing.assert_array_equal(st[key].cpu().numpy(), ost[key], err_msg=key)
    np.testing.assert_array_equal(storage_to_logical(st["v"], vcx.value_token()), ost["v"])
    np.testing.assert_array_equal(st["means"].view(torch.int16).cpu().numpy().view(np.uint16), ost["means"])
    out = forward_prepared(st)
    for r0, r1 in ((0, 3), (N // 2 - 1, N // 2 + 1), (N - 3, N)):
        _, pd = vcx.forward(st["q"], st["k"], st["v"], st["qs"], st["ks"], st["vs"], st["means"], True, True, 1,
                            D ** -0.5, p_rows=(r0, r1))
        eout, ecodes = o.reference(ost, query_indices=np.arange(r0, r1), return_codes=True)
        np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
        got = out[:, :, r0:r1].float().cpu().numpy()
        err, bound = output_bound(got, eout)
        assert np.all(err <= bound), (r0, float((err - bound).max()))
        assert cosine(got, eout) >= 0.9999


BLOCK = [  # B, H, Nq, Nk, D, dtype
    (1, 2, 300, 700, 128, torch.bfloat16),
    (2, 1, 129, 257, 64, torch.float16),
    (1, 1, 1, 1, 128, torch.bfloat16),
    # the deferred mean term: 36 tiles (two full 16-tile chunks, the 17-slot ring wraps
    # twice), a chunk that ends on the last tile, and a last tile that opens a chunk
    (1, 1, 64, 4500, 128, torch.bfloat16),
    (1, 2, 40, 2048, 64, torch.float16),
    (1, 1, 33, 2049, 128, torch.bfloat16),
]


@pytest.mark.parametrize("case", BLOCK, ids=lambda c: _ids(c))
def test_attention_block_scales_p_bytes_and_output(case):
    # v_scale_mode="block" (reference vc.py:161; preprocess.cu:24-57): every tile's
    # contribution (PV + mass * mean) is scaled by that tile's per-channel V scale.
    B, H, Nq, Nk, D, dt = case
    _print_case("attention block scales", case)
    q, k, v = make_qkv(B, H, Nq, Nk, D, dt, seed=11, kind="outlier")
    st = o.prepare(bits(q), bits(k), bits(v), v_smooth=True, v_scale_mode="block", dtype=dtype_name(dt))
    assert st["vs"].ndim == 4
    tok = vcx.value_token()
    to = _to_dev
    v8 = to(logical_to_storage(st["v"], tok)).view(torch.float8_e4m3fn)
    out, pd = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]),
                          to(st["means"]).view(torch.float16), True, True, st["output_type"], st["scale"],
                          channel_scale=False, p_rows=(0, Nq))
    eout, ecodes = o.reference(st, return_codes=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound), float((err - bound).max())
    assert cosine(got, eout) >= 0.9999


def test_sageattn_vc_block_scale_end_to_end():
    from sageattention_local import sageattn_vc
    q, k, v = make_qkv(1, 2, 257, 400, 128, torch.bfloat16, seed=5, kind="outlier")
    _print_case("sageattn_vc block scales")
    out = sageattn_vc(*(x.to(DEV) for x in (q, k, v)), v_smooth=True, v_scale_mode="block").float().cpu().numpy()
    st = _oracle_state(q, k, v, True, torch.bfloat16)
    stb = o.prepare(bits(q), bits(k), bits(v), v_smooth=True, v_scale_mode="block", dtype="bfloat16")
    eout = o.reference(stb)
    err, bound = output_bound(out, eout)
    assert np.all(err <= bound)
    assert cosine(out, eout) >= 0.9999
    # the channel-scale output of the same inputs is close but not identical
    assert not np.array_equal(eout, o.reference(st))


def test_main_config_all_heads_payloads_and_sampled_rows():
    # The benchmark's main workload in full ([1,28,37741,128] bf16, smoothing off): every
    # payload byte and scale of all 28 heads, and the P bytes / output of 8 query rows
    # spread over every head (first, last and ragged-block rows included).
    from bench import make_inputs
    B, H, N, D = 1, 28, 37741, 128
    _print_case("main config, all heads, bench inputs")
    q, k, v = make_inputs(B, H, N, D, "normal")
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    q8, qs, k8, ks, _ = vcx.prepare_qk(qd, kd)
    v8, vs, _ = vcx.prepare_v(vd)
    st = _oracle_state(q, k, v, False, torch.bfloat16)
    np.testing.assert_array_equal(q8.cpu().numpy(), st["q"])
    np.testing.assert_array_equal(k8.cpu().numpy(), st["k"])
    np.testing.assert_array_equal(qs.cpu().numpy(), st["qs"])
    np.testing.assert_array_equal(ks.cpu().numpy(), st["ks"])
    np.testing.assert_array_equal(storage_to_logical(v8, vcx.value_token()), st["v"])
    np.testing.assert_array_equal(vs.cpu().numpy(), st["vs"])
    rows = np.array([0, 1, 4711, 18870, 29999, 37631, 37700, 37740])
    # both ExpCast encodes: unfused, and folded (the reference's default mode, which the
    # benchmark times)
    for affine in (False, True):
        out = vcx.forward(q8, k8, v8, qs, ks, vs, None, True, False, 1, D ** -0.5, affine=affine)
        eout, ecodes = o.reference(st, query_indices=rows, return_codes=True, affine=affine)
        for r0 in (0, 37700):  # the P-dump variant takes one contiguous row range per launch
            r1 = r0 + 41 if r0 else 2
            _, pd = vcx.forward(q8, k8, v8, qs, ks, vs, None, True, False, 1, D ** -0.5, affine=affine,
                                p_rows=(r0, r1))
            sel = [i for i, r in enumerate(rows) if r0 <= r < r1]
            np.testing.assert_array_equal(pd.cpu().numpy()[:, :, rows[sel] - r0], ecodes[:, :, sel])
        got = out[:, :, rows].float().cpu().numpy()
        err, bound = output_bound(got, eout)
        assert np.all(err <= bound), float((err - bound).max())
        assert cosine(got, eout) >= 0.9999


CONTROL = [  # B, H, Nq, Nk, D, dtype, V mode
    (1, 2, 2048, 2048, 128, torch.bfloat16, "none"),
    (1, 1, 1, 1, 128, torch.bfloat16, "none"),
    (2, 3, 65, 129, 64, torch.float16, "channel"),
    (1, 1, 129, 513, 64, torch.bfloat16, "channel"),
    (1, 2, 257, 385, 128, torch.float16, "channel"),
    (1, 2, 300, 700, 128, torch.bfloat16, "block"),
]


@pytest.mark.parametrize("case", CONTROL, ids=lambda c: _ids(c[:6]) + "_" + c[6])
def test_control_path_p_bytes_and_output(case):
    # expcast=False, the Sage FP8 control path (vc_reference.py:58-66, attn_utils.cuh:355-455):
    # P = E4M3(exp2(fmaf(base, factor, -m'))) with the correctly rounded binary32 exp2:
    # every P byte equals the oracle's.
    B, H, Nq, Nk, D, dt, vmode = case
    _print_case("control path", case)
    smooth = vmode != "none"
    q, k, v = make_qkv(B, H, Nq, Nk, D, dt, seed=13, kind="outlier" if smooth else "normal")
    st = o.prepare(bits(q), bits(k), bits(v), expcast=False, v_smooth=smooth,
                   v_scale_mode="block" if vmode == "block" else "channel", dtype=dtype_name(dt))
    assert st["expcast"] is False
    to = _to_dev
    v8 = to(logical_to_storage(st["v"], vcx.value_token())).view(torch.float8_e4m3fn)
    means = to(st["means"]).view(torch.float16) if smooth else None
    out, pd = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]), means,
                          False, smooth, st["output_type"], st["scale"], channel_scale=vmode != "block",
                          p_rows=(0, Nq))
    eout, ecodes = o.reference(st, return_codes=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound), float((err - bound).max())
    assert cosine(got, eout) >= 0.9999
    out2 = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]), means,
                       False, smooth, st["output_type"], st["scale"], channel_scale=vmode != "block")
    assert torch.equal(out2, out)


@pytest.mark.parametrize("dim", [64, 128])
def test_control_path_far_logits_p_bytes_and_output(dim):
    # Q scaled by 25: many scores lie more than 103 nats below their row maximum, so p =
    # exp2(x) is 0 or subnormal; the window check must still give the oracle's bytes (and not
    # fall back to the binary64 recheck on every tile).
    _print_case("control path far logits", dim)
    q, k, v = make_qkv(1, 2, 200, 700, dim, torch.bfloat16, seed=29)
    q = (q.float() * 25).to(torch.bfloat16)
    st = o.prepare(bits(q), bits(k), bits(v), expcast=False, v_smooth=False, dtype="bfloat16")
    to = _to_dev
    v8 = to(logical_to_storage(st["v"], vcx.value_token())).view(torch.float8_e4m3fn)
    out, pd = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]), None,
                          False, False, st["output_type"], st["scale"], p_rows=(0, 200))
    eout, ecodes = o.reference(st, return_codes=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    assert (ecodes == 0).mean() > 0.5  # most probabilities round to byte 0
    got = out.float().cpu().numpy()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound), float((err - bound).max())
    assert cosine(got, eout) >= 0.9999


def test_control_path_uniform_attention_known_answer_and_end_to_end():
    # scripts/validate_sage_vc.py:161-182: q = k = 0 gives every key p = 2^8.807 (byte 0x7E),
    # so the output is the decoded V mean times 448 / 2^8.807f.
    from sageattention_local import sageattn_vc
    q = torch.zeros(1, 1, 65, 128, device=DEV, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 513, 128, device=DEV, dtype=torch.bfloat16)
    v = ((torch.arange(513, device=DEV).view(1, 1, 513, 1) / 128 - 2)
         * torch.linspace(.5, 1.5, 128, device=DEV) + torch.arange(128, device=DEV).remainder(11) * .125)
    v = v.to(torch.bfloat16).contiguous()
    _print_case("control path uniform")
    v8, vs, _ = vcx.prepare_v(v)
    dec = torch.from_numpy(o.e4m3_decode(storage_to_logical(v8, vcx.value_token())[..., :513]))
    weight = 448.0 / 2.0 ** float(np.float32(8.807))
    expected = (dec.double().mean(-1) * vs.cpu().double() * weight).unsqueeze(2).expand(1, 1, 65, 128)
    out = sageattn_vc(q, k, v, expcast=False, v_smooth=False)
    torch.testing.assert_close(out.double().cpu(), expected, rtol=0.004, atol=0.004)
    # random inputs through the public entry against the oracle
    q, k, v = make_qkv(1, 2, 300, 500, 128, torch.bfloat16, seed=21, kind="outlier")
    got = sageattn_vc(*(x.to(DEV) for x in (q, k, v)), expcast=False, v_smooth=True).float().cpu().numpy()
    eout = o.reference(o.prepare(bits(q), bits(k), bits(v), expcast=False, v_smooth=True, dtype="bfloat16"))
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound)
    assert cosine(got, eout) >= 0.9999


def _f32_bits(lo, hi):
    """Bits of every binary32 value in [lo, hi] (same sign), ascending in magnitude."""
    a, b = (int(np.float32(v).view(np.uint32)) for v in (lo, hi))
    return min(a, b), max(a, b)


@pytest.mark.parametrize("last_tile", [False, True])
def test_control_probability_bytes_exhaustive(last_tile):
    # Every binary32 input of the control path's P byte (x <= 8.8125 = the offset maximum 8.807
    # plus its rounding): E4M3(RN_f32(exp2(x))) from the fused kernel's device function vs the
    # oracle (binary64 exp2 rechecked in binary128), all 4.7e8 inputs with 2^-24 <= |x| <= 11 /
    # 8.8125. Outside that range the byte is fixed: 1.0 (0x38) for |x| < 2^-24, 0 for x < -11.
    chunk = 1 << 25
    mism = 0
    for lo, hi in ((2.0 ** -24, 8.8125), (-(2.0 ** -24), -11.0)):
        a, b = _f32_bits(lo, hi)
        for first in range(a, b + 1, chunk):
            n = min(chunk, b + 1 - first)
            _print_case("control probability sweep", last_tile, hex(first), n)
            x = torch.arange(first, first + n, dtype=torch.int64, device=DEV).to(torch.int32).view(torch.float32)
            got = vcx.fp8_exp2_codes(x, last_tile).cpu().numpy()
            exp = o.fp8_exp2_sweep(first, n)
            bad = np.flatnonzero(got != exp)
            assert bad.size == 0, (hex(first + int(bad[0])), int(got[bad[0]]), int(exp[bad[0]]), bad.size)
            mism += bad.size
    # the two fixed ranges, checked on the device (2.8e9 inputs)
    for (lo, hi), want in ((_f32_bits(0.0, 2.0 ** -24 * 0.99999994), 0x38), (_f32_bits(-0.0, -(2.0 ** -24) * 0.99999994), 0x38),
                           (_f32_bits(-11.000001, -3.4028235e38), 0)):
        for first in range(lo, hi + 1, 1 << 28):
            n = min(1 << 28, hi + 1 - first)
            x = torch.arange(first, first + n, dtype=torch.int64, device=DEV).to(torch.int32).view(torch.float32)
            y = vcx.fp8_exp2_codes(x, last_tile)
            assert bool((y == want).all()), (hex(first), want)
    assert vcx.fp8_exp2_codes(torch.tensor([-np.inf], device=DEV), last_tile).item() == 0
    assert mism == 0


FOLDED = [  # B, H, Nq, Nk, D, dtype, q/k magnitude (large values push |m'| past 128: group fallback)
    (1, 2, 2048, 2048, 128, torch.bfloat16, 1.0),
    (1, 2, 257, 385, 128, torch.float16, 1.0),
    (1, 1, 63, 127, 64, torch.bfloat16, 1.0),
    (1, 1, 1, 1, 128, torch.bfloat16, 1.0),
    (1, 2, 300, 700, 64, torch.bfloat16, 6.0),
]


@pytest.mark.parametrize("case", FOLDED, ids=lambda c: _ids(c[:6]) + f"_x{c[6]:g}")
def test_folded_encode_p_bytes_bit_exact_and_output(case):
    # The reference's default ExpCast kernel without block values (vc_math.cuh:16-111,
    # FoldAffine): bytes RNE(fmaf(base, RN(scale*A), fmaf(-m', A, B))), with the unfused
    # bytes for every 16-row group and tile in which some |m'| > 128.
    B, H, Nq, Nk, D, dt, mag = case
    _print_case("folded encode", case)
    q, k, v = make_qkv(B, H, Nq, Nk, D, dt, seed=17)
    q, k = (x.float().mul(mag).to(dt) for x in (q, k))
    st = _oracle_state(q, k, v, False, dt)
    to = _to_dev
    v8 = to(logical_to_storage(st["v"], vcx.value_token())).view(torch.float8_e4m3fn)
    out, pd = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]), None,
                          True, False, st["output_type"], st["scale"], affine=True, p_rows=(0, Nq))
    eout, ecodes = o.reference(st, return_codes=True, affine=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out.float().cpu().numpy()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound), float((err - bound).max())
    assert cosine(got, eout) >= 0.9999
    out2 = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]), None,
                       True, False, st["output_type"], st["scale"], affine=True)
    assert torch.equal(out2, out)


@pytest.mark.parametrize("extreme, code", [((), FOLD_CODE_FOLDED), ((3,), FOLD_CODE_UNFUSED), ((19,), FOLD_CODE_FOLDED)])
def test_folded_encode_known_answer_and_group_fallback_on_gpu(extreme, code):
    # helpers.folded_encode_payload: key 96 of row 0 is 115 folded / 116 unfused; an extreme
    # row in the same 16-row group (row 3) forces the unfused byte, one in the next group
    # (row 19) does not.
    s = folded_encode_payload(extreme_rows=extreme)
    _print_case("folded encode KA", extreme)
    to = _to_dev
    v8 = to(logical_to_storage(s["v"], vcx.value_token())).view(torch.float8_e4m3fn)
    _, pd = vcx.forward(to(s["q"]), to(s["k"]), v8, to(s["qs"]), to(s["ks"]), to(s["vs"]), None,
                        True, False, 1, s["scale"], affine=True, p_rows=(0, 32))
    got = pd.cpu().numpy()
    assert got[0, 0, 0, 96] == code and got[0, 0, 0, 45] == 120
    _, ecodes = o.reference(s, return_codes=True, affine=True)
    np.testing.assert_array_equal(got, ecodes)


@pytest.mark.parametrize("factor", [1e4, 1e-36], ids=["large", "tiny"])
def test_folded_encode_known_answer_when_the_head_precheck_fails(factor):
    # The kernel first tests the fold conditions for a whole head at once (the extreme K
    # scales, a |logit| bound per row). Scaling the last tile's K scales by 1e4 (the bound
    # passes 128) or 1e-36 (the smallest scale is subnormal) fails that test, so tile 0
    # tests the conditions itself: they hold there, and key 96 keeps its folded byte.
    s = folded_encode_payload()
    s["ks"] = s["ks"].copy()
    s["ks"][:, :, 4:8] *= np.float32(factor)
    _print_case("folded encode KA, head precheck fails", factor)
    to = _to_dev
    v8 = to(logical_to_storage(s["v"], vcx.value_token())).view(torch.float8_e4m3fn)
    _, pd = vcx.forward(to(s["q"]), to(s["k"]), v8, to(s["qs"]), to(s["ks"]), to(s["vs"]), None,
                        True, False, 1, s["scale"], affine=True, p_rows=(0, 32))
    got = pd.cpu().numpy()
    assert got[0, 0, 0, 96] == FOLD_CODE_FOLDED and got[0, 0, 0, 45] == 120
    _, ecodes = o.reference(s, return_codes=True, affine=True)
    np.testing.assert_array_equal(got, ecodes)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("factor", [10.0, 300.0, 1e-36], ids=["moderate", "large", "tiny"])
def test_folded_encode_per_tile_conditions_with_k_scale_outliers(dim, factor):
    # The K scales of tile 2 (of 8) multiplied by `factor`: the head-wide test of the fold
    # conditions fails, and every tile tests them itself. moderate: every |m'| stays <= 128
    # (all tiles fold); large: tile 2's logits pass 128, so from tile 2 on every row group
    # takes the unfused bytes; tiny: tile 2's scale is subnormal (tile 2 unfused only).
    # P bytes exact against the oracle, output within the bound.
    q, k, v = make_qkv(1, 2, 160, 900, dim, torch.bfloat16, seed=23)
    st = _oracle_state(q, k, v, False, torch.bfloat16)
    st["ks"] = st["ks"].copy()
    st["ks"][:, :, 8:12] *= np.float32(factor)
    _print_case("fold conditions per tile", dim, factor)
    to = _to_dev
    v8 = to(logical_to_storage(st["v"], vcx.value_token())).view(torch.float8_e4m3fn)
    out, pd = vcx.forward(to(st["q"]), to(st["k"]), v8, to(st["qs"]), to(st["ks"]), to(st["vs"]), None,
                          True, False, st["output_type"], st["scale"], affine=True, p_rows=(0, 160))
    eout, ecodes = o.reference(st, return_codes=True, affine=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out.float().cpu().numpy()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound), float((err - bound).max())


def test_deferred_mean_restore_rising_maximum_across_chunks():
    # Smoothing path: the block-mean restore is applied every 16 tiles from the rows' tile
    # masses, rescaled whenever the running maximum moves. Scores that grow with the key
    # index move every row's maximum in every tile (40 tiles: two full chunks and a partial
    # one), and clustered V gives large block means: the output must still meet the bound
    # against the oracle, and the P bytes stay exact.
    B, H, N, D = 1, 2, 40 * 128 - 37, 128
    g = torch.Generator().manual_seed(77)
    q = (torch.randn(B, H, 160, D, generator=g) * 0.3 + 1.0).to(torch.bfloat16)
    ramp = torch.linspace(0.0, 1.0, N).view(1, 1, N, 1)
    k = (torch.randn(B, H, N, D, generator=g) * 0.3 + ramp * 0.5).to(torch.bfloat16)
    cent = torch.randn(B, H, 8, D, generator=g) * 3.0
    v = (cent[:, :, torch.randint(0, 8, (N,), generator=g)] + 0.2 * torch.randn(B, H, N, D, generator=g)).to(
        torch.bfloat16)
    _print_case("deferred restore rising max", N)
    st = _oracle_state(q, k, v, True, torch.bfloat16)
    tok = vcx.value_token()
    v8 = _to_dev(logical_to_storage(st["v"], tok)).view(torch.float8_e4m3fn)
    out, pd = vcx.forward(_to_dev(st["q"]), _to_dev(st["k"]), v8, _to_dev(st["qs"]), _to_dev(st["ks"]),
                          _to_dev(st["vs"]), _to_dev(st["means"]).view(torch.float16), True, True,
                          st["output_type"], st["scale"], p_rows=(0, 160))
    eout, ecodes = o.reference(st, return_codes=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out.float().cpu().numpy()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound), float((err - bound).max())
    assert cosine(got, eout) >= 0.9999


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_int8_quantizers_on_every_input_bit_pattern(dt):
    # Every finite 16-bit pattern of the input dtype, as Q and as K (after centring): the
    # quantizers' reciprocal-and-FMA quotient must give the bytes of the oracle's IEEE
    # division under every group scale these rows produce.
    bits_all = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = torch.from_numpy(bits_all.view(np.int16).copy()).view(dt)
    x = torch.where(torch.isfinite(x), x, torch.zeros_like(x))
    x = x.view(1, 1, 512, 128)
    perm = torch.randperm(512, generator=torch.Generator().manual_seed(3))
    for name, t in (("ordered", x), ("shuffled rows", x[:, :, perm].contiguous())):
        _print_case("every bit pattern", dt, name)
        q8, qs, k8, ks, km = vcx.prepare_qk(t.to(DEV), t.to(DEV))
        nm = dtype_name(dt)
        eq8, eqs = o.quant_q(bits(t), nm)
        ekm = o.k_mean(bits(t), None, nm)
        ek8, eks = o.quant_k(bits(t), ekm, None, nm)
        np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint32), eqs.view(np.uint32))
        np.testing.assert_array_equal(q8.cpu().numpy(), eq8)
        np.testing.assert_array_equal(ks.cpu().numpy().view(np.uint32), eks.view(np.uint32))
        np.testing.assert_array_equal(k8.cpu().numpy(), ek8)
