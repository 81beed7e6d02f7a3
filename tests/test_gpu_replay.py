"""The four replay arms on the GPU (reference src/vc_attention/replay.py:17):
every arm runs the hip backend on the same inputs and stays close to the FP32 dense
softmax; the report is strict JSON."""
import json

import pytest
import torch

from vc_attention import replay

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("clustered", [False, True])
def test_four_arms_against_fp32_softmax(tmp_path, clustered):
    print("case: replay arms, clustered =", clustered, flush=True)
    out = tmp_path / "replay.json"
    args = replay.parse_args(["synthetic", "--tokens", "1536", "--heads", "2", "--dim", "128", "--queries", "128:256",
                              "--repeats", "2", "--output", str(out)] + (["--clustered"] if clustered else []))
    report = replay.run(args)
    assert json.loads(out.read_text()) == json.loads(json.dumps(report))
    assert report["shape_q"] == [1, 2, 256, 128] and report["shape_k"] == [1, 2, 1536, 128]
    assert report["query_range"] == [128, 384]
    # the backend's known answers ran first and are recorded (reference replay.py:66-73,134)
    assert report["preflight"]["preflight"] == "passed"
    for name, row in report["arms"].items():
        m = row["metrics"]
        # INT8 QK + FP8 P/V: a few percent relative RMSE against the unquantized softmax
        assert m["relative_rmse"] < 0.08 and m["cosine"] > 0.996, (name, m)
        assert row["config"]["backend"] == "hip" and len(row["wall_ms"]) == 2
    if clustered:
        # smoothing removes the per-cluster offsets from the E4M3 residuals
        arms = report["arms"]
        assert arms["v_smooth"]["metrics"]["relative_rmse"] < arms["expcast"]["metrics"]["relative_rmse"]


def test_captured_file_round_trip(tmp_path):
    print("case: replay capture", flush=True)
    q, k, v = replay.synthetic_inputs(640, 1, 64, 5, False)
    path = tmp_path / "qkv.pt"
    torch.save({"q": q.to(torch.float16), "k": k.to(torch.float16), "v": v.to(torch.float16),
                "metadata": {"scale": 0.11}}, path)
    out = tmp_path / "r.json"
    report = replay.run(replay.parse_args(["capture", str(path), "--dtype", "float16", "--queries", "0:0",
                                           "--repeats", "1", "--warmup", "0", "--output", str(out)]))
    assert report["source"]["kind"] == "captured_qkv" and report["scale"] == 0.11
    assert report["shape_q"] == [1, 1, 640, 64]
    assert all(row["metrics"]["cosine"] > 0.99 for row in report["arms"].values())
