"""vcx_prepare_qk_int8_noalloc (the allocation-free variant of vcx_prepare_qk_int8, no
counterpart in the reference): through the C ABI, on two calls in a row (the second with a
smaller input), its outputs equal those of vcx_prepare_qk_int8 with a caller workspace."""
import ctypes

import pytest
import torch

import vcx
from helpers import make_qkv

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
_DT = {torch.float16: 0, torch.bfloat16: 1}


def _outputs(q, k):
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    return (torch.empty((B, H, Nq, D), dtype=torch.int8, device=DEV),
            torch.empty((B, H, (Nq + 63) // 64 * 32), dtype=torch.float32, device=DEV),
            torch.empty((B, H, Nk, D), dtype=torch.int8, device=DEV),
            torch.empty((B, H, (Nk + 127) // 128 * 4), dtype=torch.float32, device=DEV),
            torch.empty((B, H, 1, D), dtype=q.dtype, device=DEV))


def _noalloc(q, k, perm):
    outs = _outputs(q, k)
    B, H, Nq, D = q.shape
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    rc = vcx.lib().vcx_prepare_qk_int8_noalloc(p(q), p(k), _DT[q.dtype], B, H, Nq, k.shape[2], D,
                                               *q.stride()[:3], *k.stride()[:3], p(perm), *(p(t) for t in outs),
                                               stream)
    assert rc == 0, vcx.lib().vcx_last_error().decode()
    return outs


def _inputs(B, H, Nq, Nk, D, dt, seed, nhd=False, permuted=False):
    q, k, _ = make_qkv(B, H, Nq, Nk, D, dt, seed=seed, kind="outlier")
    q, k = q.to(DEV), k.to(DEV)
    if nhd:  # strided HND views of NHD storage
        q, k = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q, k))
    perm = None
    if permuted:
        g = torch.Generator().manual_seed(seed)
        perm = torch.stack([torch.randperm(Nk, generator=g) for _ in range(B * H)]).view(B, H, Nk).to(DEV)
    return q, k, perm


def test_noalloc_matches_the_workspace_entry_point_on_two_calls():
    # first the main configuration's shape (8.5 MB of scratch), then a smaller one that
    # reuses (and only partly overwrites) the same scratch
    for case in ((1, 28, 37741, 37741, 128, torch.bfloat16, 3, False, True),
                 (2, 3, 257, 1000, 64, torch.float16, 4, True, False)):
        print("case: noalloc", case, flush=True)
        q, k, perm = _inputs(*case)
        want = vcx.prepare_qk(q, k, perm)
        got = _noalloc(q, k, perm)
        torch.cuda.synchronize()
        for name, a, b in zip(("q8", "qs", "k8", "ks", "km"), want, got):
            assert torch.equal(a, b), name


def test_noalloc_rejects_shapes_beyond_its_scratch_before_any_launch():
    # 64 heads x 782 tiles x 128 channels of fp64 sums = 51 MB > 32 MiB
    L = vcx.lib()
    rc = L.vcx_prepare_qk_int8_noalloc(None, None, 1, 1, 64, 128, 100000, 128, 0, 0, 128, 0, 0, 128, None,
                                       None, None, None, None, None, None)
    assert rc == 1 and "scratch" in L.vcx_last_error().decode()
    assert vcx.NOALLOC_SCRATCH_BYTES == 32 << 20
