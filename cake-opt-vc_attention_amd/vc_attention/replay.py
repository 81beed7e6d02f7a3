"""Same-input accuracy replay of the hip backend's four numerical arms.

Each arm of ``ARMS`` (the reference's arm table, src/vc_attention/replay.py:17: Sage FP8
probabilities without smoothing, ExpCast, V smoothing, both) runs
``vc_attention.attention`` with ``Config(backend="hip")`` on one input set, and is scored
against an FP32 dense softmax of the very same (already FP16/BF16-rounded) values. The
error measures keep the reference's definitions (replay.py:20-32): RMSE, RMSE relative to
the reference's RMS, largest absolute difference, cosine similarity.

Inputs come from one of two sources:

* ``synthetic``: Q, K, V ~ N(0,1) drawn from one CPU ``torch.Generator`` in that order;
  ``--clustered`` then replaces V by one of 8 per-head centroids (scale 8) plus 0.1 V,
  drawn in the order of the reference's generator (replay.py:41-48) so that every machine
  sees the same numbers;
* ``capture``: a Q/K/V file (``torch.load(weights_only=True)``) checked as
  scripts/profile_int8_h200.py:54-75 checks captured MiniMax tensors.

Only query rows are selected (``--queries START:COUNT``, START a 128-row boundary, COUNT 0
for all); every key/value token stays, because a cropped context is another attention.
Arms are timed with device events on the current stream, repeats rotating the arm order;
grouping runs on every call.

    python -m vc_attention.replay synthetic --tokens 8192 --heads 4 --clustered --queries 0:1024
    python -m vc_attention.replay capture qkv.pt --layout NHD --output report.json
"""
import argparse
import hashlib
import json
import math
import platform
import statistics
from dataclasses import asdict
from pathlib import Path

import torch

from .core import Config, attention
from .hip_backend import preflight

# arm name -> (v_smooth, expcast)
ARMS = {"fp8_control": (False, False), "expcast": (False, True), "v_smooth": (True, False), "combined": (True, True)}


def error_metrics(actual, reference):
    """Float64 error of `actual` against `reference`: rmse, relative_rmse (over the
    reference's RMS), max_abs and cosine."""
    a = actual.detach().double().reshape(-1)
    r = reference.detach().double().reshape(-1)
    if not bool(torch.isfinite(a).all()):
        raise ValueError("Nonfinite attention output")
    norm = torch.linalg.vector_norm
    diff, ref_norm, act_norm = norm(a - r).item(), norm(r).item(), norm(a).item()
    return {
        "rmse": diff / math.sqrt(a.numel()),
        "relative_rmse": diff / max(ref_norm, 1e-15 * math.sqrt(a.numel())),
        "max_abs": (a - r).abs().max().item(),
        "cosine": torch.dot(a, r).item() / max(act_norm * ref_norm, 1e-300),
    }


def synthetic_inputs(tokens, heads, dim, seed, clustered):
    """[1, heads, tokens, dim] float32 Q, K, V from a seeded CPU generator."""
    gen = torch.Generator().manual_seed(seed)
    shape = (1, heads, tokens, dim)
    q, k, v = (torch.randn(shape, generator=gen) for _ in "qkv")
    if not clustered:
        return q, k, v
    centroids = torch.randn((1, heads, 8, dim), generator=gen) * 8
    which = torch.randint(0, 8, (1, heads, tokens, 1), generator=gen)
    return q, k, torch.take_along_dim(centroids, which, dim=2) + 0.1 * v


def load_capture(path, layout="HND"):
    """Captured Q/K/V (scripts/profile_int8_h200.py:54-75): a dict with 4-D FP16/BF16 tensors
    q, k, v of one MHA shape (D 64/128, finite, nonempty) and optional ``metadata``; ``scale``
    comes from metadata when present. Returns ((q, k, v) in HND, scale, source record)."""
    path = Path(path)
    data = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(data, dict) or not all(isinstance(data.get(n), torch.Tensor) for n in ("q", "k", "v")):
        raise ValueError("QKV file must contain tensors under q, k, v")
    qkv = tuple(data[n] for n in ("q", "k", "v"))
    if any(x.ndim != 4 for x in qkv):
        raise ValueError("Captured Q/K/V must be four-dimensional")
    if layout not in ("HND", "NHD"):
        raise ValueError("layout must be HND or NHD")
    if layout == "NHD":
        qkv = tuple(x.transpose(1, 2) for x in qkv)
    q, k, v = qkv
    if (q.dtype not in (torch.float16, torch.bfloat16) or any(x.dtype != q.dtype for x in qkv)
            or k.shape != v.shape or q.shape[:2] != k.shape[:2] or q.shape[-1] != k.shape[-1]
            or q.shape[-1] not in (64, 128) or any(x.numel() == 0 for x in qkv)):
        raise ValueError("Captured QKV require matching FP16/BF16 MHA, D64/128, nonempty shapes")
    if not all(bool(torch.isfinite(x).all()) for x in qkv):
        raise ValueError("Captured QKV contain NaN/Inf")
    metadata = data.get("metadata") or {}
    if not isinstance(metadata, dict):
        raise ValueError("metadata must be a dict")
    scale = float(metadata.get("scale", q.shape[-1] ** -0.5))
    source = {"kind": "captured_qkv", "file": str(path.resolve()), "layout": layout,
              "sha256": hashlib.sha256(path.read_bytes()).hexdigest(), "metadata": metadata}
    return tuple(x.contiguous() for x in (q, k, v)), scale, source


@torch.no_grad()
def exact_attention(q, k, v, scale, chunk=256):
    """FP32 dense softmax(Q K^T * scale) V over all keys, in query chunks (never N x N)."""
    kt = k.float().transpose(-1, -2).contiguous()
    vf = v.float().contiguous()
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    for begin in range(0, q.shape[-2], chunk):
        qc = q[..., begin:begin + chunk, :].float().contiguous()
        s = torch.matmul(qc, kt) * scale
        out[..., begin:begin + chunk, :] = torch.matmul(torch.softmax(s, dim=-1), vf)
    return out


def parse_queries(text):
    """'START:COUNT' -> (start, count); count 0 selects every row from start."""
    try:
        start, count = (int(x) for x in text.split(":"))
    except ValueError:
        raise argparse.ArgumentTypeError("expected START:COUNT") from None
    if start < 0 or count < 0:
        raise argparse.ArgumentTypeError("START and COUNT must be non-negative")
    return start, count


def select_queries(q, start, count):
    """Query rows [start, start + count) (count 0: to the end); start on a 128-row block."""
    n = q.shape[-2]
    if start % 128 or start >= n:
        raise ValueError(f"query start {start} must be a 128-row block boundary below {n}")
    end = n if count == 0 else min(n, start + count)
    return q[..., start:end, :], [start, end]


def time_arms(calls, device, warmup, repeats):
    """Milliseconds per call of every arm: events on the current stream of `device`; repeat r
    runs the arms starting from the r-th (rotating order). Returns (times, last results)."""
    names = list(calls)
    for _ in range(warmup):
        for name in names:
            calls[name]()
    times = {name: [] for name in names}
    results = {}
    for rep in range(repeats):
        for name in names[rep % len(names):] + names[:rep % len(names)]:
            if device.type == "cuda":
                begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                begin.record()
                results[name] = calls[name]()
                end.record()
                end.synchronize()
                times[name].append(begin.elapsed_time(end))
            else:
                results[name] = calls[name]()
                times[name].append(float("nan"))
    return times, results


def run(args):
    """Run every arm on the same inputs; write the JSON report to args.output and return it."""
    device = torch.device(args.device)
    dtype = {"bfloat16": torch.bfloat16, "float16": torch.float16}[args.dtype]
    if args.source == "capture":
        (q, k, v), scale, source = load_capture(args.file, args.layout)
    else:
        q, k, v = synthetic_inputs(args.tokens, args.heads, args.dim, args.seed, args.clustered)
        source = {"kind": "synthetic_clustered" if args.clustered else "synthetic_gaussian", "seed": args.seed}
        scale = args.dim ** -0.5
    q, query_range = select_queries(q, *args.queries)
    # the backend's known answers before any arm, recorded in the report (reference
    # replay.py:66-73,134); the argument and input checks above run first
    preflight_result = preflight(args.device) if device.type == "cuda" else None
    q, k, v = (x.to(dtype).to(device).contiguous() for x in (q, k, v))
    exact = exact_attention(q, k, v, scale)
    configs = {name: Config(backend="hip", qk_format="int8", q_block=64, k_quant_block=128, kv_block=128,
                            qk_hadamard=False, v_smooth=smooth, expcast=cast, clusters=args.clusters,
                            iterations=args.iterations)
               for name, (smooth, cast) in ARMS.items()}
    calls = {name: (lambda c=cfg: attention(q, k, v, c, scale=scale)[0]) for name, cfg in configs.items()}
    times, results = time_arms(calls, device, args.warmup, args.repeats)
    report = {
        "status": "exploratory",
        "source": source,
        "device": str(device),
        "device_name": torch.cuda.get_device_name(device) if device.type == "cuda" else platform.processor(),
        "torch": torch.__version__,
        "host": platform.platform(),
        "preflight": preflight_result,
        "dtype": args.dtype,
        "shape_q": list(q.shape),
        "shape_k": list(k.shape),
        "scale": scale,
        "query_range": query_range,
        "reference": "FP32 dense softmax on the same input values",
        "full_kv_context": True,
        "timing": "device events per call on the current stream, rotating arm order, grouping included",
        "warmup": args.warmup,
        "repeats": args.repeats,
        "arms": {name: {"metrics": error_metrics(results[name].float(), exact), "wall_ms": times[name],
                        "median_ms": statistics.median(times[name]), "config": asdict(configs[name])}
                 for name in calls},
    }
    out = Path(args.output)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(report, indent=2, allow_nan=False) + "\n", encoding="utf-8")
    return report


def _positive(text):
    value = int(text)
    if value < 1:
        raise argparse.ArgumentTypeError("must be >= 1")
    return value


def _non_negative(text):
    value = int(text)
    if value < 0:
        raise argparse.ArgumentTypeError("must be >= 0")
    return value


def build_parser():
    common = argparse.ArgumentParser(add_help=False)
    common.add_argument("--device", default="cuda:0")
    common.add_argument("--dtype", choices=("bfloat16", "float16"), default="bfloat16",
                        help="the hip backend's input type; the FP32 reference reads the rounded values")
    common.add_argument("--clusters", type=_positive, default=8)
    common.add_argument("--iterations", type=_positive, default=2)
    common.add_argument("--queries", type=parse_queries, default=(0, 256), metavar="START:COUNT",
                        help="query rows to score (COUNT 0 = all); every key is always kept")
    common.add_argument("--warmup", type=_non_negative, default=1)
    common.add_argument("--repeats", type=_positive, default=3)
    common.add_argument("--output", default="vc-replay-hip.json")
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = parser.add_subparsers(dest="source", required=True)
    syn = sub.add_parser("synthetic", parents=[common], help="seeded Gaussian (or clustered-V) inputs")
    syn.add_argument("--tokens", type=_positive, default=2048)
    syn.add_argument("--heads", type=_positive, default=2)
    syn.add_argument("--dim", type=int, choices=(64, 128), default=128)
    syn.add_argument("--seed", type=int, default=20260917)
    syn.add_argument("--clustered", action="store_true")
    cap = sub.add_parser("capture", parents=[common], help="a captured Q/K/V file")
    cap.add_argument("file")
    cap.add_argument("--layout", choices=("HND", "NHD"), default="HND")
    return parser


def parse_args(argv=None):
    return build_parser().parse_args(argv)


def main(argv=None):
    report = run(parse_args(argv))
    print(json.dumps({name: row["metrics"] for name, row in report["arms"].items()}, indent=2))
    return report


if __name__ == "__main__":
    main()
