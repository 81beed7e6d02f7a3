"""vc_attention.attention(Config(backend="hip")) over a denoising-step schedule against the
oracle (reference src/vc_attention/core.py:197-226 LayoutCache, :263-371 attention;
tests/test_core.py:96-123).

One request runs eight steps of one layer with V changing at every step:
  steps 0 and 4 regroup (refresh_interval 4; step 4 warm-starts from step 0's centers),
  steps 1-3 and 5 reuse the cached permutation with the current V's means and residuals,
  steps 6 and 7 are past the smoothing window (ceil(8 * 0.75) = 6): no block values, the
  folded ExpCast encode, K and V still gathered by the cached permutation.
Each step is compared with the oracle fed the same permutation: the GPU permutation equals
the oracle's warm-started grouping, every sampled row's P bytes are equal, and the output
meets helpers.output_bound and cosine >= 0.9999.
"""
import numpy as np
import pytest
import torch

import vcx
from helpers import bits, cosine, dtype_name, make_qkv, output_bound
from oracle import vc_oracle as o
from vc_attention import Config, LayoutCache, attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _cfg(clusters=8):
    return Config(backend="hip", qk_format="int8", q_block=64, k_quant_block=128, kv_block=128, qk_hadamard=False,
                  expcast=True, v_smooth=True, active_fraction=0.75, refresh_interval=4, clusters=clusters,
                  iterations=2)


def _step_value(v0, step, dt):
    g = torch.Generator().manual_seed(100 + step)
    return (v0.float() + 0.25 * step * torch.randn(v0.shape, generator=g)).to(dt)


@pytest.mark.parametrize("D,dt,clusters", [(128, torch.bfloat16, 8), (64, torch.float16, 16)])
def test_denoising_schedule_matches_the_oracle_step_by_step(D, dt, clusters):
    print("case: schedule", D, dt, clusters, flush=True)
    cfg = _cfg(clusters)
    cache = LayoutCache(cfg)
    q, k, v0 = make_qkv(1, 2, 300, 700, D, dt, seed=31, kind="outlier")
    rows = np.unique(np.r_[np.arange(0, 300, 37), 299])
    perm = centers = None
    for step in range(8):
        v = _step_value(v0, step, dt)
        out, counters = attention(q.to(DEV), k.to(DEV), v.to(DEV), cfg, cache=cache, step=step, total_steps=8,
                                  request_id="req", layer_id=3)
        active, refresh = step < 6, step in (0, 4)
        assert counters["smoothing_active"] == active and counters["layout_refreshed"] == refresh, step
        if refresh:  # the oracle's grouping, warm-started from the previous refresh's centers
            perm, _, _, centers = o.group_values(bits(v), clusters, 2, dtype_name(dt), centers_in=centers,
                                                 return_next=True)
        gpu_perm = cache._layers[3].permutation
        np.testing.assert_array_equal(gpu_perm.cpu().numpy(), perm)
        st = o.prepare(bits(q), bits(k), bits(v), v_smooth=active, permutation=perm, dtype=dtype_name(dt))
        eout, ecodes = o.reference(st, query_indices=rows, return_codes=True, affine=not active)
        got = out.float().cpu().numpy()[:, :, rows]
        err, bound = output_bound(got, eout)
        assert np.all(err <= bound), (step, float((err - bound).max()))
        assert cosine(got, eout) >= 0.9999, step
        # the same payloads through the diagnostic kernel: every sampled row's P bytes
        q8, qs, k8, ks, _ = vcx.prepare_qk(q.to(DEV), k.to(DEV), gpu_perm)
        v8, vs, means = vcx.prepare_v(v.to(DEV), gpu_perm, smooth=active)
        for r in rows:
            _, pd = vcx.forward(q8, k8, v8, qs, ks, vs, means, True, active, st["output_type"], st["scale"],
                                affine=not active, p_rows=(int(r), int(r) + 1))
            np.testing.assert_array_equal(pd.cpu().numpy()[:, :, 0], ecodes[:, :, list(rows).index(r)])


def test_reused_layout_recomputes_current_means_and_residuals():
    # tests/test_core.py:116-123: at a reuse step, V + 7 moves the output by 7. With INT8 QK
    # and E4M3 residuals the identity holds to the output rounding (bf16 ulp at 7 is 2^-5)
    # plus the fp16 rounding of the shifted block means; each output also matches the oracle.
    cfg = _cfg()
    cache = LayoutCache(cfg)
    q, k, v = make_qkv(1, 2, 130, 513, 128, torch.bfloat16, seed=7, kind="outlier")
    a, _ = attention(q.to(DEV), k.to(DEV), v.to(DEV), cfg, cache=cache, step=0, total_steps=20, request_id="x")
    v7 = (v.float() + 7).to(torch.bfloat16)
    b, counters = attention(q.to(DEV), k.to(DEV), v7.to(DEV), cfg, cache=cache, step=1, total_steps=20,
                            request_id="x")
    assert counters["smoothing_active"] and not counters["layout_refreshed"]
    a, b = a.float().cpu(), b.float().cpu()
    # half a bf16 ulp of each output (2^-8 relative) plus the block means' fp16 rounding
    assert bool(((b - (a + 7)).abs() <= 2.0 ** -8 * (b.abs() + a.abs()) + 1e-2).all())
    perm = cache._layers[0].permutation.cpu().numpy()
    st = o.prepare(bits(q), bits(k), bits(v7), v_smooth=True, permutation=perm)
    eout = o.reference(st)
    err, bound = output_bound(b.numpy(), eout)
    assert np.all(err <= bound)
