"""Timing of the chunked-prefill cache flow on one
layer: Llama-3.1-8B head shape, chunks of 4096 tokens up to 65536, through
``DropKVCache.update`` exactly as ``prefill_chunked`` drives it
(dropkv_cache.py:651-807), in the default mode (``torch.cat`` of the stored
K/V and the chunk, gather into new tensors) and in the capacity mode
(append in place, gather between preallocated buffers).

Each chunk's Q/K/V are drawn on the device before the timed region; the
model's own work (projections, the chunk's attention) is not part of the
flow.  ``python -m dropkv_amd.chunked_flow`` prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys

import torch

from .dropkv_cache import DropKVCache


def _mode(strategy: str, i: int, n: int, stored: int, chunk: int, max_kv: int) -> str:
    last = i == n - 1
    if strategy == "last_chunk":
        return "evict_accumulated" if last else "accumulate"
    if strategy == "every_chunk":
        return "single_pass" if i == 0 else "evict_accumulated"
    if last:
        return "evict_accumulated"
    return "evict_accumulated" if stored + chunk > max_kv else "accumulate"


def run_flow(cache: DropKVCache, chunks, strategy: str, max_kv: int) -> None:
    cache._evict_use_seen_tokens = strategy in ("budget", "every_chunk")
    cache._budget_max_kv_tokens = max_kv if strategy == "budget" else None
    n = len(chunks)
    try:
        for i, (q, k, v) in enumerate(chunks):
            stored = cache.key_cache[0].shape[2] if cache.key_cache else 0
            cache._prefill_mode = _mode(strategy, i, n, stored, k.shape[2], max_kv)
            cache.update(q, k, v, layer_idx=0)
    finally:
        cache._prefill_mode = "single_pass"
        cache._evict_use_seen_tokens = False
        cache._budget_max_kv_tokens = None


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--length", type=int, default=65536)
    p.add_argument("--chunk", type=int, default=4096)
    p.add_argument("--keep-ratio", type=float, default=0.1)
    p.add_argument("--max-kv", type=int, default=32768)
    p.add_argument("--reps", type=int, default=5)
    p.add_argument("--strategies", default="every_chunk,last_chunk,budget")
    args = p.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("chunked_flow needs a ROCm GPU")
    dev = torch.device("cuda:0")
    B, Hq, Hkv, D = 1, 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(0)
    chunks = []
    for s in range(0, args.length, args.chunk):
        n = min(args.chunk, args.length - s)
        chunks.append(tuple(torch.randn(B, h, n, D, device=dev, generator=g).bfloat16() for h in (Hq, Hkv, Hkv)))
    res = {}
    for strategy in args.strategies.split(","):
        for label, capacity in (("default", None), ("capacity", args.length)):
            times = []
            for rep in range(args.reps + 1):
                cache = DropKVCache(keep_ratio=args.keep_ratio, capacity=capacity)
                torch.cuda.synchronize()
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                run_flow(cache, chunks, strategy, args.max_kv)
                end.record()
                torch.cuda.synchronize()
                if rep:
                    times.append(start.elapsed_time(end))
                stored = cache.key_cache[0].shape[2]
                del cache
            res[f"{strategy}/{label}"] = {"ms_per_flow": round(statistics.median(times), 3),
                                          "ms_per_chunk": round(statistics.median(times) / len(chunks), 4),
                                          "stored_rows": stored}
            print(f"[flow] {strategy} {label}: {res[f'{strategy}/{label}']}", file=sys.stderr, flush=True)
    print(json.dumps({"workload": "chunked_llama8b_64k", "B": B, "Hq": Hq, "Hkv": Hkv, "D": D,
                      "length": args.length, "chunk": args.chunk, "keep_ratio": args.keep_ratio,
                      "max_kv_tokens": args.max_kv, "reps": args.reps,
                      "timing": "HIP events around the whole flow on the current stream (host launch work included)",
                      **res}), flush=True)


if __name__ == "__main__":
    main()
