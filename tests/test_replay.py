"""The four-arm replay tool (reference src/vc_attention/replay.py): CPU checks of its
metrics, input generator, capture loader and argument rules; the arms themselves run
under the GPU marker."""
import json
import math

import numpy as np
import pytest
import torch

from vc_attention import replay


def test_arms_match_the_reference_table():
    # replay.py:17
    assert replay.ARMS == {"fp8_control": (False, False), "expcast": (False, True), "v_smooth": (True, False),
                           "combined": (True, True)}


def test_metrics_known_values():
    ref = torch.tensor([3.0, 4.0, 0.0, 0.0])
    got = torch.tensor([3.0, 4.0, 1.0, -1.0])
    m = replay.error_metrics(got, ref)
    assert m["rmse"] == pytest.approx(math.sqrt(2 / 4))
    assert m["relative_rmse"] == pytest.approx(math.sqrt((2 / 4) / (25 / 4)))
    assert m["max_abs"] == 1.0
    assert m["cosine"] == pytest.approx(25 / (5 * math.sqrt(27)))
    with pytest.raises(ValueError, match="Nonfinite"):
        replay.error_metrics(torch.tensor([float("nan")]), torch.tensor([1.0]))


def test_synthetic_inputs_are_deterministic_and_clustered():
    a = replay.synthetic_inputs(256, 2, 64, 7, True)
    b = replay.synthetic_inputs(256, 2, 64, 7, True)
    for x, y in zip(a, b):
        assert x.shape == (1, 2, 256, 64) and torch.equal(x, y)
    v = a[2][0, 0]
    # every row lies within the 0.1-scaled noise of one of 8 centroids of scale 8
    d = torch.cdist(v, v)
    near = (d < 2.0).float().sum(-1)
    assert near.min() >= 2 and len(torch.unique((d < 2.0).float(), dim=0)) <= 8
    g = replay.synthetic_inputs(256, 2, 64, 7, False)
    assert torch.equal(g[0], a[0]) and torch.equal(g[1], a[1]) and not torch.equal(g[2], a[2])


def _save(tmp_path, name="qkv.pt", **record):
    path = tmp_path / name
    torch.save(record, path)
    return path


def test_capture_loader_accepts_hnd_and_nhd_with_metadata_scale(tmp_path):
    gen = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 2, 33, 64, generator=gen).to(torch.bfloat16) for _ in range(3))
    path = _save(tmp_path, q=q, k=k, v=v, metadata={"scale": 0.1, "layer": 3})
    (q2, k2, v2), scale, source = replay.load_capture(path)
    assert torch.equal(q2, q) and torch.equal(v2, v) and scale == 0.1
    assert source["kind"] == "captured_qkv" and len(source["sha256"]) == 64 and source["metadata"]["layer"] == 3
    nhd = _save(tmp_path, "nhd.pt", q=q.transpose(1, 2).contiguous(), k=k.transpose(1, 2).contiguous(),
                v=v.transpose(1, 2).contiguous())
    (q3, _, _), scale3, _ = replay.load_capture(nhd, "NHD")
    assert torch.equal(q3, q) and scale3 == pytest.approx(64 ** -0.5)


@pytest.mark.parametrize("record, match", [
    (dict(q=torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)), "q, k, v"),
    (dict(q=torch.zeros(1, 4, 64, dtype=torch.bfloat16), k=torch.zeros(1, 4, 64, dtype=torch.bfloat16),
          v=torch.zeros(1, 4, 64, dtype=torch.bfloat16)), "four-dimensional"),
    (dict(q=torch.zeros(1, 1, 4, 64), k=torch.zeros(1, 1, 4, 64), v=torch.zeros(1, 1, 4, 64)), "FP16/BF16"),
    (dict(q=torch.zeros(1, 1, 4, 96, dtype=torch.float16), k=torch.zeros(1, 1, 4, 96, dtype=torch.float16),
          v=torch.zeros(1, 1, 4, 96, dtype=torch.float16)), "D64/128"),
    (dict(q=torch.zeros(1, 2, 4, 64, dtype=torch.float16), k=torch.zeros(1, 1, 4, 64, dtype=torch.float16),
          v=torch.zeros(1, 1, 4, 64, dtype=torch.float16)), "MHA"),
    (dict(q=torch.full((1, 1, 4, 64), float("nan"), dtype=torch.float16), k=torch.zeros(1, 1, 4, 64, dtype=torch.float16),
          v=torch.zeros(1, 1, 4, 64, dtype=torch.float16)), "NaN"),
])
def test_capture_loader_rejections(tmp_path, record, match):
    with pytest.raises(ValueError, match=match):
        replay.load_capture(_save(tmp_path, **record))


def test_exact_attention_matches_a_float64_softmax():
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, 2, n, 64, generator=gen) for n in (70, 300, 300))
    got = replay.exact_attention(q, k, v, 0.125, chunk=32).double()
    s = (q.double() @ k.double().transpose(-1, -2)) * 0.125
    want = torch.softmax(s, -1) @ v.double()
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_synthetic_draw_order_is_q_k_v_then_centroids_then_assignment():
    # the reference's generator order (replay.py:41-48), restated with an explicit gather
    gen = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(1, 3, 40, 64, generator=gen) for _ in range(3))
    cent = torch.randn(1, 3, 8, 64, generator=gen) * 8
    ids = torch.randint(0, 8, (1, 3, 40, 1), generator=gen)
    want = torch.gather(cent, 2, ids.expand(1, 3, 40, 64)) + 0.1 * v
    got = replay.synthetic_inputs(40, 3, 64, 11, True)
    assert torch.equal(got[0], q) and torch.equal(got[1], k) and torch.equal(got[2], want)


def test_argument_rules(tmp_path):
    with pytest.raises(SystemExit):
        replay.parse_args(["synthetic", "--tokens", "0"])
    with pytest.raises(SystemExit):
        replay.parse_args(["synthetic", "--queries", "0:-1"])
    with pytest.raises(SystemExit):
        replay.parse_args(["synthetic", "--queries", "12"])
    with pytest.raises(SystemExit):
        replay.parse_args([])
    a = replay.parse_args(["capture", "x.pt", "--layout", "NHD", "--queries", "128:0"])
    assert a.source == "capture" and a.file == "x.pt" and a.queries == (128, 0)
    args = replay.parse_args(["synthetic", "--queries", "64:128", "--output", str(tmp_path / "r.json")])
    with pytest.raises(ValueError, match="128-row block"):
        replay.run(args)


def test_select_queries_keeps_every_key_row_range():
    q = torch.zeros(1, 1, 600, 64)
    sel, rng = replay.select_queries(q, 128, 256)
    assert sel.shape[-2] == 256 and rng == [128, 384]
    sel, rng = replay.select_queries(q, 512, 0)
    assert sel.shape[-2] == 88 and rng == [512, 600]
    with pytest.raises(ValueError):
        replay.select_queries(q, 640, 0)


def test_time_arms_rotates_the_order_on_the_cpu():
    seen = []
    calls = {n: (lambda n=n: seen.append(n) or torch.zeros(1)) for n in "abcd"}
    times, results = replay.time_arms(calls, torch.device("cpu"), warmup=1, repeats=3)
    assert seen[:4] == list("abcd") and seen[4:8] == list("abcd") and seen[8:12] == list("bcda")
    assert seen[12:] == list("cdab") and all(len(t) == 3 for t in times.values()) and set(results) == set("abcd")
