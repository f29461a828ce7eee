"""End-to-end harness: a Qwen2-0.5B-architecture model with random-init bf16
weights, a uniform-random prompt, DropKV eviction at prefill, then greedy
decode on the compressed cache.

The reference has no such script; its README and integration tests drive a
pretrained Qwen2-0.5B through the patched Transformers (README.md:96-140,
tests/test_dropkv_triton.py:763-825).  With no network for checkpoints, the
same architecture is built from its public configuration and initialised
from a seed.  The model is the installed Transformers' ``Qwen2ForCausalLM``
(SDPA attention); the cache is :class:`dropkv_amd.hf_cache.DropKVCache`,
which evicts each layer's K/V with the HIP layer-call during prefill.

Run ``python -m dropkv_amd.e2e_qwen2`` on a GPU; it prints one JSON line with
the prefill time and the decode rate on the compressed cache -- decoded by
:class:`dropkv_amd.decode.CompressedDecoder` (preallocated buffers, one HIP
graph per step) and, for comparison, eagerly through Transformers -- and the
same figures with the uncompressed ``DynamicCache``.
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
import time

import torch

from . import hf_cache
from .decode import CompressedDecoder

# Qwen2-0.5B architecture (public model configuration).
QWEN2_05B = dict(
    vocab_size=151936,
    hidden_size=896,
    intermediate_size=4864,
    num_hidden_layers=24,
    num_attention_heads=14,
    num_key_value_heads=2,
    max_position_embeddings=32768,
    rope_theta=1e6,
    rms_norm_eps=1e-6,
    tie_word_embeddings=True,
)


def make_config(**overrides):
    """A ``Qwen2Config`` for the architecture above (fields overridable),
    with SDPA attention."""
    from transformers import Qwen2Config

    spec = dict(QWEN2_05B)
    spec.update(overrides)
    theta = spec.pop("rope_theta")
    cfg = Qwen2Config(rope_parameters={"rope_theta": theta, "rope_type": "default"}, **spec)
    cfg._attn_implementation = "sdpa"
    return cfg


def build_model(cfg, device, dtype=torch.bfloat16, seed: int = 0):
    """Random-init ``Qwen2ForCausalLM`` (the Transformers initialiser, seeded)."""
    from transformers import Qwen2ForCausalLM

    torch.manual_seed(seed)
    with torch.device(device):
        model = Qwen2ForCausalLM(cfg)
    return model.to(dtype).eval()


def random_prompt(vocab: int, length: int, batch: int = 1, seed: int = 1, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (batch, length), generator=g).to(device)


@torch.no_grad()
def prefill(model, input_ids, cache):
    """One forward over the prompt with ``cache``; returns the greedy next
    token [B, 1].  Only the last position's logits are computed."""
    with hf_cache.query_capture():
        out = model(input_ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
    return out.logits[:, -1].argmax(-1, keepdim=True)


@torch.no_grad()
def greedy_decode(model, cache, token, steps: int):
    """``steps`` greedy decode steps on ``cache``; returns the tokens
    [B, steps].  Tokens stay on the device (no host round trip per step)."""
    toks = []
    with hf_cache.query_capture():
        for _ in range(steps):
            out = model(token, past_key_values=cache, use_cache=True, logits_to_keep=1)
            token = out.logits[:, -1].argmax(-1, keepdim=True)
            toks.append(token)
    return torch.cat(toks, dim=1)


def _timed(fn):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    r = fn()
    torch.cuda.synchronize()
    return r, (time.perf_counter() - t0) * 1e3


def run(args) -> dict:
    from transformers import DynamicCache

    dev = torch.device("cuda:0")
    cfg = make_config(num_hidden_layers=args.layers)
    model = build_model(cfg, dev, seed=args.seed)
    ids = random_prompt(cfg.vocab_size, args.prompt, seed=args.seed + 1, device=dev)

    def make_cache(kind):
        if kind == "dropkv":
            return hf_cache.DropKVCache(cfg, keep_ratio=args.keep_ratio, window_size=args.window,
                                        kernel_size=args.kernel_size)
        return DynamicCache(config=cfg)

    res = {}
    kinds = ("dropkv", "dropkv_eager", "dynamic") if args.compare else ("dropkv",)
    for kind in kinds:
        pre_ms, dec_ms, setup_ms = [], [], []
        for rep in range(args.warmup + args.reps):
            cache = make_cache("dynamic" if kind == "dynamic" else "dropkv")
            tok, t_pre = _timed(lambda: prefill(model, ids, cache))
            if kind == "dropkv":
                dec, t_setup = _timed(lambda: CompressedDecoder(model, cache, args.decode))
                out, t_dec = _timed(lambda: dec.generate(tok, args.decode))
                stored, logical = int(dec.n_rows[0]), int(dec.pos[0, 0])
                del dec
            else:
                t_setup = 0.0
                out, t_dec = _timed(lambda: greedy_decode(model, cache, tok, args.decode))
                stored, logical = cache.layers[0].keys.shape[-2], cache.get_seq_length()
            if rep >= args.warmup:
                pre_ms.append(t_pre)
                dec_ms.append(t_dec)
                setup_ms.append(t_setup)
            print(f"[e2e] {kind} rep {rep}: prefill {t_pre:.1f} ms, decode setup {t_setup:.1f} ms, "
                  f"decode {args.decode} steps {t_dec:.1f} ms", file=sys.stderr, flush=True)
        res[kind] = {
            "prefill_ms": statistics.median(pre_ms),
            "decode_tok_s": args.decode / (statistics.median(dec_ms) / 1e3),
            "stored_kv_rows_layer0": stored,
            "logical_length": logical,
        }
        if kind == "dropkv":
            res[kind]["decode"] = "CompressedDecoder: HIP graph per step, dropkv_decode_attention"
            res[kind]["decode_setup_ms"] = statistics.median(setup_ms)
        else:
            res[kind]["decode"] = "eager Transformers forward per step (SDPA, torch.cat append)"
        del cache
        torch.cuda.empty_cache()
    return {
        "workload": "qwen2_0.5b_e2e",
        "data": "synthetic: random-init bf16 weights, uniform random prompt ids",
        "config": {"layers": args.layers, "hidden": cfg.hidden_size, "Hq": cfg.num_attention_heads,
                   "Hkv": cfg.num_key_value_heads, "D": cfg.hidden_size // cfg.num_attention_heads,
                   "vocab": cfg.vocab_size, "prompt": args.prompt, "decode_steps": args.decode,
                   "keep_ratio": args.keep_ratio, "window": args.window, "kernel_size": args.kernel_size,
                   "attn": "sdpa", "dtype": "bf16"},
        "reps": args.reps,
        **res,
    }


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--prompt", type=int, default=16384)
    p.add_argument("--decode", type=int, default=256)
    p.add_argument("--layers", type=int, default=QWEN2_05B["num_hidden_layers"])
    p.add_argument("--keep-ratio", type=float, default=0.1)
    p.add_argument("--window", type=int, default=8)
    p.add_argument("--kernel-size", type=int, default=11)
    p.add_argument("--reps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-compare", dest="compare", action="store_false",
                   help="skip the uncompressed DynamicCache comparison")
    args = p.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("e2e_qwen2 needs a ROCm GPU")
    print(json.dumps(run(args)), flush=True)


if __name__ == "__main__":
    main()
