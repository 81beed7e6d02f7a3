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
