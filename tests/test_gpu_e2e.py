"""BASELINE configuration 4 at its configured size on the GPU: the
Qwen2-0.5B architecture (24 layers, hidden 896, Hq 14, Hkv 2, D 64, vocab
151936, random-init bf16 weights), a 16384-token uniform-random prompt
through ``hf_cache.DropKVCache(0.1, 8, 11)``, then decode on the compressed
cache.

The reference drives a pretrained Qwen2-0.5B through its patched
Transformers (tests/test_dropkv_triton.py:757-842, :1083-1160); with no
checkpoint offline, the same architecture is initialised from a seed.

* Layers 0, 11 and 23: the kept set against the oracle
  (``dropkv_scores_reference(match_pytorch_precision=True)``, pool, protect,
  top-k) on the very (query, key, value) the layer received: tie-aware
  overlap >= 0.999; the binding scores (>= 0.1x the keep threshold) within
  2e-2, fewer than 1e-3 of them beyond 1e-3; the compressed K/V equal to a
  gather by the kept indices, bit for bit.
* 256 decode steps (the configuration's decode length) of
  ``CompressedDecoder`` (HIP graph per step) and of the eager bf16
  Transformers decode on the same cache, both against a float32
  copy of the model attending over the same stored rows (at the logical RoPE
  position): the decoder must be as close to the float32 logits as the eager
  bf16 decode is (bf16 rounding differences compound over 24 random-init
  layers to a few percent of the logits, so the two bf16 paths are compared
  through the float32 one rather than with each other).
"""

import copy

import pytest
import torch

pytest.importorskip("transformers")

from conftest import assert_binding_scores  # noqa: E402
from oracle import dropkv_ref as R  # noqa: E402

pytestmark = pytest.mark.gpu

CHECK_LAYERS = (0, 11, 23)
DECODE_STEPS = 256


def test_c4_qwen2_05b_16k_prefill_and_decode(gpu, monkeypatch):
    from dropkv_amd import hf_cache
    from dropkv_amd.decode import CompressedDecoder
    from dropkv_amd.e2e_qwen2 import build_model, make_config, prefill, random_prompt
    from dropkv_amd.hf_query import query_capture

    cfg = make_config()
    assert (cfg.num_hidden_layers, cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads,
            cfg.vocab_size) == (24, 896, 14, 2, 151936)
    model = build_model(cfg, gpu, dtype=torch.bfloat16, seed=0)
    L, ratio, W, ks = 16384, 0.1, 8, 11
    keep = int(ratio * L)
    assert keep == 1638
    rec, calls = {}, []
    real = hf_cache._evict

    def recording(q, k, v, window, kernel_size, kk, use_triton):
        out = real(q, k, v, window, kernel_size, kk, use_triton)
        layer = len(calls)
        calls.append(kk)
        if layer in CHECK_LAYERS:
            rec[layer] = (q[:, :, -window:].cpu(), k.cpu(), v.cpu(), [t.cpu() for t in out], window, kernel_size)
        return out

    monkeypatch.setattr(hf_cache, "_evict", recording)
    cache = hf_cache.DropKVCache(cfg, keep_ratio=ratio, window_size=W, kernel_size=ks)
    ids = random_prompt(cfg.vocab_size, L, seed=1, device=gpu)
    print("[c4] prefill 16384 tokens", flush=True)
    tok = prefill(model, ids, cache)
    torch.cuda.synchronize()
    monkeypatch.setattr(hf_cache, "_evict", real)
    assert calls == [keep] * 24
    assert cache.get_seq_length() == L and all(cache.stored_length(i) == keep for i in range(24))

    for layer in CHECK_LAYERS:
        qt, kb, vb, (idx, kc, vc), window, kernel_size = rec[layer]
        assert idx.shape == (1, 2, keep) and torch.equal(idx, torch.sort(idx, dim=-1).values)
        s_ref = R.dropkv_scores_reference(qt, kb, vb, window, match_pytorch_precision=True)
        pooled = R.pool_protect(s_ref.clone(), kernel_size, window)
        overlap, unexcused = R.index_overlap(idx, R.topk_sorted(pooled, keep), pooled)
        assert overlap >= 0.999, (layer, overlap, unexcused)
        from dropkv_amd import ops
        got = ops.scores(qt.to(gpu), kb.to(gpu), vb.to(gpu), window, p_round=True).cpu()
        stats = assert_binding_scores(got, s_ref, pooled, keep, qt, kb, vb, window, torch.bfloat16, 2e-2, 1e-3,
                                      1e-3)
        print(f"[c4 layer {layer}] overlap {overlap}, binding keys {stats[0]}, worst rel {stats[1]:.2e}",
              flush=True)
        rk, rv = R.gather_compressed(kb, vb, idx)
        assert torch.equal(kc, rk) and torch.equal(vc, rv)
        assert torch.equal(cache.layers[layer].keys.cpu(), kc)

    # Decode on the compressed cache: the graph-replayed decoder and the eager
    # bf16 decode, each against the float32 model over the same stored rows.
    from transformers import DynamicCache
    print(f"[c4] {DECODE_STEPS} decode steps", flush=True)
    dec = CompressedDecoder(model, cache, max_new_tokens=DECODE_STEPS, use_graph=True)
    model32 = copy.deepcopy(model).float()
    dc32 = DynamicCache(config=cfg)
    for i, lay in enumerate(cache.layers):
        dc32.update(lay.keys.float().clone(), lay.values.float().clone(), i)
    e_dec, e_eager = [], []
    with torch.no_grad(), query_capture():
        for t in range(DECODE_STEPS):
            eager = model(tok, past_key_values=cache, use_cache=True, logits_to_keep=1).logits.float()
            got = dec.step(tok).clone().float()
            ref = model32(tok, past_key_values=dc32, use_cache=True, logits_to_keep=1,
                          position_ids=torch.tensor([[L + t]], device=gpu)).logits
            e_dec.append((got - ref).abs())
            e_eager.append((eager - ref).abs())
            if t % 32 == 0 or t == DECODE_STEPS - 1:
                print(f"[c4 decode {t}] decoder vs fp32: max {e_dec[-1].max().item():.4f} mean "
                      f"{e_dec[-1].mean().item():.5f}; eager bf16 vs fp32: max {e_eager[-1].max().item():.4f} "
                      f"mean {e_eager[-1].mean().item():.5f}; max|ref| {ref.abs().max().item():.3f}", flush=True)
            tok = ref[:, -1].argmax(-1, keepdim=True)
    e_dec, e_eager = torch.stack(e_dec), torch.stack(e_eager)
    assert e_dec.mean() <= 1.25 * e_eager.mean(), (e_dec.mean().item(), e_eager.mean().item())
    assert e_dec.max() <= 1.5 * e_eager.max(), (e_dec.max().item(), e_eager.max().item())
    del model32, dc32
    assert int(dec.n_rows[0]) == cache.stored_length(0) == keep + DECODE_STEPS
    assert int(dec.pos[0, 0]) == cache.get_seq_length() == L + DECODE_STEPS
    del dec, cache, model
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
