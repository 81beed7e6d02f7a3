"""GPU parity of the Hadamard Q/K rotation (libvcx, through its C ABI) against the CPU oracle.

Bit-exact: the rotated INT8 Q/K payloads and scales (vcx_prepare_qk_int8_rotated) and the
binary32 outputs of the generic preprocessing (vcx_preprocess_qk, the reference's
preprocess_qk), whose cases follow tests/test_paper_alignment.py:124-150 (D 37/64/128,
fp32/fp16/bf16, the four k_smooth x rotate combinations, non-contiguous input, a side
stream); P bytes of the fused kernel on rotated payloads; the vc_attention hip backend
with qk_hadamard=True end to end.
"""
import numpy as np
import pytest
import torch

import vcx
from helpers import bits, cosine, dtype_name, make_qkv, output_bound
from oracle import vc_oracle as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _print_case(*args):
    print("case:", *args, flush=True)


SHAPES = [  # B, H, Nq, Nk, D, dtype
    (1, 2, 2048, 2048, 128, torch.bfloat16),
    (2, 3, 65, 129, 64, torch.float16),
    (1, 2, 257, 385, 128, torch.float16),
    (1, 1, 63, 127, 64, torch.bfloat16),
    (1, 1, 1, 1, 128, torch.bfloat16),
]


@pytest.mark.parametrize("kind", ["normal", "outlier"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B%dH%dq%dk%dD%d" % s[:5])
def test_rotated_int8_payloads_bit_exact(shape, kind):
    B, H, Nq, Nk, D, dt = shape
    _print_case("rotated prepare_qk", shape, kind)
    q, k, _ = make_qkv(B, H, Nq, Nk, D, dt, seed=12, kind=kind)
    q8, qs, k8, ks, km = vcx.prepare_qk(q.to(DEV), k.to(DEV), hadamard=True)
    name = dtype_name(dt)
    ekm = o.k_mean(bits(k), None, name)
    eq8, eqs = o.quant_q(bits(q), name, rotate=True)
    ek8, eks = o.quant_k(bits(k), ekm, None, name, rotate=True)
    np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint32), eqs.view(np.uint32))
    np.testing.assert_array_equal(q8.cpu().numpy(), eq8)
    np.testing.assert_array_equal(ks.cpu().numpy().view(np.uint32), eks.view(np.uint32))
    np.testing.assert_array_equal(k8.cpu().numpy(), ek8)


def test_rotated_int8_strided_nhd_and_permutation():
    B, H, N, D = 1, 3, 333, 128
    q, k, _ = make_qkv(B, H, N, N, D, torch.bfloat16, seed=3, kind="outlier")
    g = torch.Generator().manual_seed(4)
    perm = torch.stack([torch.randperm(N, generator=g) for _ in range(B * H)]).view(B, H, N)
    qn, kn = (x.transpose(1, 2).contiguous().to(DEV) for x in (q, k))
    q8, qs, k8, ks, _ = vcx.prepare_qk(qn.transpose(1, 2), kn.transpose(1, 2), perm.to(DEV), hadamard=True)
    ekm = o.k_mean(bits(k), perm.numpy())
    ek8, eks = o.quant_k(bits(k), ekm, perm.numpy(), rotate=True)
    eq8, eqs = o.quant_q(bits(q), rotate=True)
    np.testing.assert_array_equal(q8.cpu().numpy(), eq8)
    np.testing.assert_array_equal(k8.cpu().numpy(), ek8)
    np.testing.assert_array_equal(ks.cpu().numpy().view(np.uint32), eks.view(np.uint32))
    np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint32), eqs.view(np.uint32))


def _explicit_hadamard(width):
    i = np.arange(width)
    pop = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    return torch.from_numpy((-1.0) ** pop / np.sqrt(width))


@pytest.mark.parametrize("dim", [1, 16, 37, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("k_smooth,rotate", [(False, False), (False, True), (True, False), (True, True)])
def test_preprocess_qk_bit_exact_and_matrix_oracle(dim, dtype, k_smooth, rotate):
    # tests/test_paper_alignment.py:124-150
    _print_case("preprocess_qk", dim, dtype, k_smooth, rotate)
    gen = torch.Generator().manual_seed(14)
    q, k = [torch.randn(2, 2, n, dim, generator=gen) for n in (13, 35)]
    k += torch.linspace(-2, 2, dim)
    q, k = q.to(dtype), k.to(dtype)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        # non-contiguous inputs, on a side stream
        qd, kd = [torch.stack([x.to(DEV), x.to(DEV)], -1)[..., 0] for x in (q, k)]
        qo, ko = vcx.preprocess_qk(qd, kd, k_smooth, rotate)
        consumed = [x + 1 for x in (qo, ko)]
    stream.synchronize()
    name = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}[dtype]
    arg = (lambda x: x.numpy()) if dtype == torch.float32 else bits
    eq, ek = o.preprocess_qk(arg(q), arg(k), k_smooth=k_smooth, hadamard=rotate, dtype=name)
    np.testing.assert_array_equal(qo.cpu().numpy(), eq)
    np.testing.assert_array_equal(ko.cpu().numpy(), ek)
    mq, mk = q.double(), k.double()
    if k_smooth:
        mk = mk - mk.mean(-2, keepdim=True)
    if rotate:
        width = 1 << (dim - 1).bit_length()
        m = _explicit_hadamard(width)
        mq = torch.nn.functional.pad(mq, (0, width - dim)) @ m
        mk = torch.nn.functional.pad(mk, (0, width - dim)) @ m
    for got, want in zip(consumed, (mq, mk)):
        torch.testing.assert_close(got.cpu().double(), want + 1, atol=3e-6, rtol=3e-5)
    torch.testing.assert_close(qd.cpu(), q, atol=0, rtol=0)
    torch.testing.assert_close(kd.cpu(), k, atol=0, rtol=0)


def test_preprocess_qk_long_sequence_bit_exact():
    # many tiles: the mean's per-tile then over-tiles order on a 37741-key head
    q, k, _ = make_qkv(1, 2, 1000, 37741, 128, torch.bfloat16, seed=5, kind="outlier")
    qo, ko = vcx.preprocess_qk(q.to(DEV), k.to(DEV), True, True)
    eq, ek = o.preprocess_qk(bits(q), bits(k), k_smooth=True, hadamard=True, dtype="bfloat16")
    np.testing.assert_array_equal(qo.cpu().numpy(), eq)
    np.testing.assert_array_equal(ko.cpu().numpy(), ek)


@pytest.mark.parametrize("shape", [(1, 2, 1024, 1024, 128), (2, 3, 65, 129, 64)], ids=["D128", "D64"])
def test_fused_kernel_on_rotated_payloads(shape):
    # P bytes bit-exact and output within the bound of the oracle on the rotated INT8 payloads
    B, H, Nq, Nk, D = shape
    q, k, v = make_qkv(B, H, Nq, Nk, D, torch.bfloat16, seed=9, kind="outlier")
    st = o.prepare(bits(q), bits(k), bits(v), v_smooth=False, qk_hadamard=True)
    q8, qs, k8, ks, _ = vcx.prepare_qk(q.to(DEV), k.to(DEV), hadamard=True)
    v8, vs, _ = vcx.prepare_v(v.to(DEV))
    np.testing.assert_array_equal(q8.cpu().numpy(), st["q"])
    np.testing.assert_array_equal(k8.cpu().numpy(), st["k"])
    out, pd = vcx.forward(q8, k8, v8, qs, ks, vs, None, True, False, 1, D ** -0.5, affine=True, p_rows=(0, Nq))
    eout, ecodes = o.reference(st, return_codes=True, affine=True)
    np.testing.assert_array_equal(pd.cpu().numpy(), ecodes)
    got = out.float().cpu().numpy()
    err, bound = output_bound(got, eout)
    assert np.all(err <= bound)
    assert cosine(got, eout) >= 0.9999


def test_vc_attention_hip_backend_with_rotation():
    from vc_attention import Config, attention
    q, k, v = (x.to(DEV) for x in make_qkv(1, 2, 512, 700, 128, torch.bfloat16, seed=2, kind="outlier"))
    cfg = Config(backend="hip", qk_format="int8", expcast=True, q_block=64, k_quant_block=128, kv_block=128,
                 qk_hadamard=True)
    out, counters = attention(q, k, v, cfg)
    assert counters["qk_hadamard"] is True
    plain, c2 = attention(q, k, v, Config(**{**cfg.__dict__, "qk_hadamard": False}))
    assert c2["qk_hadamard"] is False and not torch.equal(out, plain)
    # both are the same attention: against the FP32 dense softmax of the same inputs
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) * 128 ** -0.5
    exact = torch.matmul(torch.softmax(s, -1), v.float())
    for o_ in (out, plain):
        rel = ((o_.float() - exact).square().mean() / exact.square().mean()).sqrt().item()
        assert rel < 0.08, rel
