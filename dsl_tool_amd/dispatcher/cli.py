"""Command line over the dispatcher (commands of the reference's
dispatcher/cli.py:35-148).

    python -m dsl_tool_amd.dispatcher.cli list
    python -m dsl_tool_amd.dispatcher.cli info --kernel gemm.fp8_gemm --backend hip
    python -m dsl_tool_amd.dispatcher.cli run --kernel gemm.fp8_gemm --backend hip \\
        --input '{"shape":[128,4096],"dtype":"bfloat16","fill":"random"}' \\
        --input '{"shape":[4096,4096],"dtype":"bfloat16","fill":"random"}' \\
        --param scale_a=1.0 --param scale_b=1.0 [--raw]

``--param k=v`` values are coerced to int, then float, then bool, else kept
as strings (reference cli.py:123-144).
"""
from __future__ import annotations

import argparse
import json
import sys
from typing import Any, Dict, List, Optional

import torch

from .dispatcher import DispatchResult, KernelDispatcher, summarize_tensor


def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description="Quantized GEMM kernel dispatcher CLI")
    sub = p.add_subparsers(dest="command", required=True)
    sub.add_parser("list", help="List all registered kernels")
    pi = sub.add_parser("info", help="Show one kernel's metadata")
    pi.add_argument("--kernel", required=True)
    pi.add_argument("--backend", required=True)
    pr = sub.add_parser("run", help="Run a kernel")
    pr.add_argument("--kernel", required=True)
    pr.add_argument("--backend", required=True)
    pr.add_argument("--input", action="append", default=[], help="JSON tensor spec (repeatable)")
    pr.add_argument("--param", action="append", default=[], help="key=value (repeatable)")
    pr.add_argument("--raw", action="store_true", help="Emit full base64 JSON output")
    return p


def main(argv: Optional[List[str]] = None) -> int:
    args = build_parser().parse_args(argv)
    d = KernelDispatcher(device="cuda")
    if args.command == "list":
        print(json.dumps(d.list_kernels(), indent=2, ensure_ascii=False))
        return 0
    if args.command == "info":
        print(json.dumps(d.kernel_info(args.kernel, args.backend), indent=2, ensure_ascii=False))
        return 0
    specs = [json.loads(s) for s in args.input]
    res = d.run_from_spec(args.kernel, args.backend, tensor_specs=specs,
                          scalar_params=parse_params(args.param))
    if args.raw:
        print(json.dumps(res.to_dict(), indent=2, ensure_ascii=False))
    else:
        print_summary(res)
    return 0


def print_summary(res: DispatchResult) -> None:
    print(f"kernel  : {res.kernel_name}")
    print(f"backend : {res.backend}")
    print(f"device  : {res.device_info}")
    print(f"elapsed : {res.elapsed_ms:.3f} ms")
    outs = res.output
    if isinstance(outs, torch.Tensor):
        outs = [outs]
    if not isinstance(outs, (list, tuple)):
        print(f"output  : {outs}")
        return
    for i, o in enumerate(outs):
        if isinstance(o, torch.Tensor):
            s = summarize_tensor(o)
            label = "output" if len(outs) == 1 else f"output[{i}]"
            print(f"{label}  : shape={s['shape']} dtype={s['dtype']}  min={s['min']:.6g}  "
                  f"max={s['max']:.6g}  mean={s['mean']:.6g}  std={s['std']:.6g}")
        else:
            print(f"output[{i}]: {o}")


def parse_params(items: List[str]) -> Dict[str, Any]:
    out: Dict[str, Any] = {}
    for item in items:
        if "=" not in item:
            raise ValueError(f"Invalid --param '{item}', expected key=value")
        k, v = item.split("=", 1)
        out[k] = coerce_scalar(v)
    return out


def coerce_scalar(v: str) -> Any:
    for conv in (int, float):
        try:
            return conv(v)
        except ValueError:
            pass
    low = v.lower()
    if low in ("true", "false"):
        return low == "true"
    return v


if __name__ == "__main__":
    sys.exit(main())
