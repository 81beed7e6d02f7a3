"""Four-arm, same-input numerical replay of the hip backend.

Mirrors the reference's src/vc_attention/replay.py: the arms of replay.py:17
(``fp8_control``: no smoothing, Sage FP8 probabilities; ``expcast``;
``v_smooth``; ``combined``) run ``attention(q, k, v, Config(backend="hip", ...))``
on the same inputs and are scored against an FP32 dense softmax over the same
input values (replay.py:20-32 metrics). Inputs are either the reference's
synthetic generator (replay.py:41-48, CPU ``torch.Generator`` so every machine
draws the same numbers) or a captured QKV file loaded with
``torch.load(weights_only=True)`` under the checks of
scripts/profile_int8_h200.py:54-75.

The hip backend takes FP16/BF16 inputs, so the replay casts to ``--dtype``
(bfloat16 by default) first and the FP32 reference reads the cast values.
All K/V tokens are kept; ``--q-start``/``--q-limit`` only select query rows
(replay.py:100-105). Wall times include grouping on every call, as in the
reference ("regrouping included on every measured call").

    python -m vc_attention.replay --tokens 4096 --heads 2 --clustered --output r.json
"""
import argparse
import hashlib
import json
import math
import platform
import statistics
import time
from dataclasses import asdict
from pathlib import Path

import torch

from .core import Config, attention

ARMS = {"fp8_control": (False, False), "expcast": (False, True), "v_smooth": (True, False), "combined": (True, True)}


def metrics(actual, reference):
    """RMSE, relative RMSE, max |delta| and cosine in float64 (replay.py:20-32)."""
    x, ref = actual.double(), reference.double()
    if not bool(torch.isfinite(x).all()):
        raise ValueError("Nonfinite attention output")
    delta = x - ref
    mse = delta.square().mean().item()
    energy = ref.square().mean().item()
    return {
        "rmse": math.sqrt(mse),
        "relative_rmse": math.sqrt(mse / max(energy, 1e-30)),
        "max_abs": delta.abs().max().item(),
        "cosine": torch.nn.functional.cosine_similarity(x.flatten(), ref.flatten(), dim=0).item(),
    }


def synthetic(tokens, heads, dim, seed, clustered):
    """The reference's replay inputs (replay.py:41-48): N(0,1) Q/K/V, optionally V drawn
    around 8 per-head centroids of scale 8 with 0.1 noise."""
    generator = torch.Generator().manual_seed(seed)
    q, k, v = [torch.randn((1, heads, tokens, dim), generator=generator) for _ in range(3)]
    if clustered:
        centers = torch.randn((1, heads, 8, dim), generator=generator) * 8
        ids = torch.randint(0, 8, (1, heads, tokens, 1), generator=generator).expand_as(v)
        v = centers.gather(-2, ids) + 0.1 * v
    return q, k, v


def load_capture(path, layout="HND"):
    """Captured Q/K/V (scripts/profile_int8_h200.py:54-75): a dict with 4-D FP16/BF16 tensors
    q, k, v of one MHA shape (D 64/128, finite, nonempty) and optional ``metadata``; ``scale``
    comes from metadata when present."""
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


def _synchronize(device):
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def run(args):
    """Run every arm on the same inputs; write and return the JSON report."""
    device = torch.device(args.device)
    dtype = {"bfloat16": torch.bfloat16, "float16": torch.float16}[args.dtype]
    if args.capture:
        (q, k, v), scale, source = load_capture(args.capture, args.layout)
    else:
        q, k, v = synthetic(args.tokens, args.heads, args.dim, args.seed, args.clustered)
        source = {"kind": "synthetic_clustered" if args.clustered else "synthetic_gaussian", "seed": args.seed}
        scale = args.dim ** -0.5
    if args.q_start % 128 or args.q_start >= q.shape[-2]:
        raise ValueError("q-start must be a valid 128-token block boundary")
    end = q.shape[-2] if args.q_limit == 0 else min(q.shape[-2], args.q_start + args.q_limit)
    # Keep every K/V token: a cropped context is not the attention being replayed.
    q = q[..., args.q_start:end, :]
    q, k, v = [x.to(dtype).to(device).contiguous() for x in (q, k, v)]
    exact = exact_attention(q, k, v, scale)
    configs = {
        name: Config(backend="hip", qk_format="int8", q_block=64, k_quant_block=128, kv_block=128,
                     qk_hadamard=False, v_smooth=smooth, expcast=cast, clusters=args.clusters,
                     iterations=args.iterations)
        for name, (smooth, cast) in ARMS.items()
    }
    calls = {name: (lambda cfg=cfg: attention(q, k, v, cfg, scale=scale)[0]) for name, cfg in configs.items()}
    for _ in range(args.warmup):
        for call in calls.values():
            call()
    times = {name: [] for name in calls}
    errors = {}
    for repeat in range(args.repeats):
        order = list(calls) if repeat % 2 == 0 else list(reversed(calls))
        for name in order:
            _synchronize(device)
            start = time.perf_counter()
            result = calls[name]()
            _synchronize(device)
            times[name].append((time.perf_counter() - start) * 1000)
            errors[name] = metrics(result.float(), exact)
    report = {
        "status": "exploratory",
        "source": source,
        "device": str(device),
        "device_name": torch.cuda.get_device_name(device) if device.type == "cuda" else platform.processor(),
        "torch": torch.__version__,
        "host": platform.platform(),
        "dtype": args.dtype,
        "shape_q": list(q.shape),
        "shape_k": list(k.shape),
        "scale": scale,
        "query_range": [args.q_start, end],
        "reference": "FP32 dense softmax on the same input values",
        "full_kv_context": True,
        "warmup": args.warmup,
        "repeats": args.repeats,
        "scope": "isolated attention; grouping included on every measured call",
        "arms": {
            name: {"metrics": errors[name], "wall_ms": times[name], "median_ms": statistics.median(times[name]),
                   "config": asdict(configs[name])}
            for name in calls
        },
    }
    output = Path(args.output)
    output.parent.mkdir(parents=True, exist_ok=True)
    output.write_text(json.dumps(report, indent=2, allow_nan=False) + "\n", encoding="utf-8")
    return report


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--capture")
    parser.add_argument("--layout", choices=("HND", "NHD"), default="HND")
    parser.add_argument("--device", default="cuda:0")
    parser.add_argument("--dtype", choices=("bfloat16", "float16"), default="bfloat16")
    parser.add_argument("--tokens", type=int, default=1024)
    parser.add_argument("--heads", type=int, default=2)
    parser.add_argument("--dim", type=int, default=128)
    parser.add_argument("--seed", type=int, default=20260917)
    parser.add_argument("--clustered", action="store_true")
    parser.add_argument("--clusters", type=int, default=8)
    parser.add_argument("--iterations", type=int, default=2)
    parser.add_argument("--q-start", type=int, default=0)
    parser.add_argument("--q-limit", type=int, default=128, help="0 = all queries; all KV tokens are always retained")
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--repeats", type=int, default=3)
    parser.add_argument("--output", default="vc-replay.json")
    args = parser.parse_args(argv)
    if min(args.tokens, args.heads, args.dim, args.repeats) < 1 or min(args.warmup, args.q_start, args.q_limit) < 0:
        parser.error("Invalid dimension/count")
    return args


def main(argv=None):
    report = run(parse_args(argv))
    print(json.dumps({name: row["metrics"] for name, row in report["arms"].items()}, indent=2))
    return report


if __name__ == "__main__":
    main()
