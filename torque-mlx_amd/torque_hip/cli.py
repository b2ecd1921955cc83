"""``python -m torque_hip benchmark {synthetic,qwen-decode}`` (reference cli.py:65-152, 369-428)."""

from __future__ import annotations

import argparse
import json

from torque_hip.benchmarking import run_synthetic_decode_benchmark
from torque_hip.cache_hip import SUPPORTED_DECODE_STRATEGIES
from torque_hip.qwen_benchmark import run_qwen_decode_runtime_benchmark


def _print_json(payload: dict[str, object]) -> None:
    print(json.dumps(payload, indent=2, sort_keys=True))


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(prog="torque-hip", description="Benchmark the MI355X packed KV-cache decode path.")
    subparsers = parser.add_subparsers(dest="command", required=True)
    benchmark_parser = subparsers.add_parser("benchmark", help="Run decode-path benchmarks.")
    bench = benchmark_parser.add_subparsers(dest="benchmark_command", required=True)

    synthetic = bench.add_parser("synthetic", help="Synthetic packed decode benchmark.")
    synthetic.add_argument("--seq-len", type=int, default=512)
    synthetic.add_argument("--head-dim", type=int, default=128)
    synthetic.add_argument("--kv-heads", type=int, default=8)
    synthetic.add_argument("--bit-width", type=int, default=4)
    synthetic.add_argument("--seed", type=int, default=0)
    synthetic.add_argument("--rotation-seed", type=int)

    qwen = bench.add_parser("qwen-decode", help="KV-growing decode loop with Qwen model geometry.")
    qwen.add_argument("--model-dir", required=True)
    qwen.add_argument("--prefill-tokens", type=int, default=2048)
    qwen.add_argument("--decode-steps", type=int, default=128)
    qwen.add_argument("--seed", type=int, default=0)
    qwen.add_argument("--bit-width", type=int)
    qwen.add_argument("--rotation-seed", type=int, default=0)
    qwen.add_argument("--decode-strategy", default="split_batched", choices=SUPPORTED_DECODE_STRATEGIES)
    qwen.add_argument("--decode-tail-capacity", type=int)
    return parser


def main(argv: list[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    if args.command == "benchmark" and args.benchmark_command == "synthetic":
        _print_json(
            run_synthetic_decode_benchmark(
                seq_len=args.seq_len,
                head_dim=args.head_dim,
                kv_heads=args.kv_heads,
                bit_width=args.bit_width,
                seed=args.seed,
                rotation_seed=args.rotation_seed,
            )
        )
        return 0
    if args.command == "benchmark" and args.benchmark_command == "qwen-decode":
        _print_json(
            run_qwen_decode_runtime_benchmark(
                model_dir=args.model_dir,
                prefill_tokens=args.prefill_tokens,
                decode_steps=args.decode_steps,
                seed=args.seed,
                bit_width=args.bit_width,
                rotation_seed=args.rotation_seed,
                decode_strategy=args.decode_strategy,
                decode_tail_capacity=args.decode_tail_capacity,
            ).to_dict()
        )
        return 0
    return 2
