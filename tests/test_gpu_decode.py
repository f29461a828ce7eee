"""Decode on the compressed cache (``dropkv_decode_attention`` and
:class:`dropkv_amd.decode.CompressedDecoder`).

The kernel is checked against a float32 PyTorch attention over the same
rows (the new token's row included), for GQA groups, both head dimensions,
an empty cache and a full buffer; the buffers must hold the new row bit for
bit afterwards, the rows past it untouched, and the row count not advanced.
The decoder (a HIP graph per step) is checked against the eager
Transformers decode over the same compressed cache, step by step with the
same input tokens, and its replays against eager runs of the same graph
inputs."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref_attention(q, k_rows, v_rows, scale):
    """q [B,Hq,1,D]; k_rows/v_rows [B,Hkv,n,D] -> [B,1,Hq,D] (float32)."""
    B, Hq, _, D = q.shape
    Hkv = k_rows.shape[1]
    g = Hq // Hkv
    k = k_rows.float().repeat_interleave(g, dim=1)
    v = v_rows.float().repeat_interleave(g, dim=1)
    s = (q.float() @ k.transpose(-1, -2)) * scale
    p = torch.softmax(s, dim=-1)
    return (p @ v).transpose(1, 2)


@pytest.mark.parametrize("B,Hq,Hkv,D,C,n,dtype", [
    (1, 14, 2, 64, 1920, 1638, torch.bfloat16),    # Qwen2-0.5B decode after eviction
    (2, 32, 8, 128, 512, 300, torch.bfloat16),     # Llama head shape, batch 2
    (1, 8, 8, 128, 256, 0, torch.bfloat16),        # MHA, empty cache: only the new row
    (1, 16, 1, 64, 128, 127, torch.float16),       # g = 16, buffer full after this step
    (1, 4, 2, 128, 4096, 4000, torch.bfloat16),    # many splits
])
def test_decode_attention_vs_torch(gpu, B, Hq, Hkv, D, C, n, dtype):
    from dropkv_amd import ops
    g = torch.Generator().manual_seed(C + n)
    kb = torch.randn(B, Hkv, C, D, generator=g).to(dtype).to(gpu)
    vb = torch.randn(B, Hkv, C, D, generator=g).to(dtype).to(gpu)
    q = torch.randn(B, Hq, 1, D, generator=g).to(dtype).to(gpu)
    kn = torch.randn(B, Hkv, 1, D, generator=g).to(dtype).to(gpu)
    vn = torch.randn(B, Hkv, 1, D, generator=g).to(dtype).to(gpu)
    k_before, v_before = kb.clone(), vb.clone()
    n_rows = torch.tensor([n], dtype=torch.int32, device=gpu)
    out = torch.empty(B, 1, Hq, D, dtype=dtype, device=gpu)
    ws = ops.decode_workspace(B, Hq, Hkv, D, C, gpu)
    scale = D ** -0.5
    ops.decode_attention(q, kn, vn, kb, vb, n_rows, scale, out, ws)
    torch.cuda.synchronize()
    k_rows = torch.cat([k_before[:, :, :n], kn], dim=2)
    v_rows = torch.cat([v_before[:, :, :n], vn], dim=2)
    ref = _ref_attention(q, k_rows, v_rows, scale)
    torch.testing.assert_close(out.float(), ref, rtol=2e-2, atol=2e-2)
    assert torch.equal(kb[:, :, n], kn[:, :, 0]) and torch.equal(vb[:, :, n], vn[:, :, 0])
    assert torch.equal(kb[:, :, :n], k_before[:, :, :n]) and torch.equal(kb[:, :, n + 1:], k_before[:, :, n + 1:])
    assert torch.equal(vb[:, :, n + 1:], v_before[:, :, n + 1:])
    assert int(n_rows.item()) == n


def test_decode_attention_strided_inputs(gpu):
    """q, k_new and v_new as the transposed projections of a decoder layer
    ([B, 1, H, D] viewed as [B, H, 1, D]); out written through strides."""
    from dropkv_amd import ops
    B, Hq, Hkv, D, C, n = 2, 14, 2, 64, 320, 200
    g = torch.Generator().manual_seed(1)
    kb = torch.randn(B, Hkv, C, D, generator=g).bfloat16().to(gpu)
    vb = torch.randn(B, Hkv, C, D, generator=g).bfloat16().to(gpu)
    q = torch.randn(B, 1, Hq, D, generator=g).bfloat16().to(gpu).transpose(1, 2)
    kn = torch.randn(B, 1, Hkv, D, generator=g).bfloat16().to(gpu).transpose(1, 2)
    vn = torch.randn(B, 1, Hkv, D, generator=g).bfloat16().to(gpu).transpose(1, 2)
    k_rows = torch.cat([kb[:, :, :n].clone(), kn], dim=2)
    v_rows = torch.cat([vb[:, :, :n].clone(), vn], dim=2)
    n_rows = torch.tensor([n], dtype=torch.int32, device=gpu)
    out = torch.empty(B, Hq, 1, D, dtype=torch.bfloat16, device=gpu).transpose(1, 2)
    ops.decode_attention(q, kn, vn, kb, vb, n_rows, D ** -0.5, out, ops.decode_workspace(B, Hq, Hkv, D, C, gpu))
    torch.testing.assert_close(out.float(), _ref_attention(q, k_rows, v_rows, D ** -0.5), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("D,Hq,Hkv", [(64, 14, 2), (128, 16, 1)])
@pytest.mark.parametrize("C,n", [
    (4160, 4159),   # 64 splits of 65 rows (two steps each, the second of one row); last row of the buffer
    (4160, 4100),
    (4160, 64),     # the new row alone in split 0's second step
    (4160, 65),     # the new row first in split 1; splits 2.. empty
    (4160, 0),      # only the new row
    (200, 130),     # 4 splits of 50 rows: one partial step each
])
def test_decode_attention_split_edges_nan_rows(gpu, D, Hq, Hkv, C, n):
    """Split rows are fixed by the capacity, so splits can run two steps,
    end in a partial step, or hold no row at all. Every buffer row from the
    new row's position on holds NaN: the rows past it are masked out of the
    logits and out of P.V (0 * NaN is NaN), and the buffer keeps them as
    they were; row n ends up holding the new row."""
    from dropkv_amd import ops
    B = 1
    g = torch.Generator().manual_seed(7 * C + n + D)
    kb = torch.randn(B, Hkv, C, D, generator=g).bfloat16()
    vb = torch.randn(B, Hkv, C, D, generator=g).bfloat16()
    kb[:, :, n:] = float("nan")
    vb[:, :, n:] = float("nan")
    kb, vb = kb.to(gpu), vb.to(gpu)
    q = torch.randn(B, Hq, 1, D, generator=g).bfloat16().to(gpu)
    kn = torch.randn(B, Hkv, 1, D, generator=g).bfloat16().to(gpu)
    vn = torch.randn(B, Hkv, 1, D, generator=g).bfloat16().to(gpu)
    k_before, v_before = kb.clone(), vb.clone()
    n_rows = torch.tensor([n], dtype=torch.int32, device=gpu)
    out = torch.empty(B, 1, Hq, D, dtype=torch.bfloat16, device=gpu)
    ops.decode_attention(q, kn, vn, kb, vb, n_rows, D ** -0.5, out, ops.decode_workspace(B, Hq, Hkv, D, C, gpu))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    ref = _ref_attention(q, torch.cat([k_before[:, :, :n], kn], dim=2), torch.cat([v_before[:, :, :n], vn], dim=2),
                         D ** -0.5)
    torch.testing.assert_close(out.float(), ref, rtol=2e-2, atol=2e-2)
    assert torch.equal(kb[:, :, n], kn[:, :, 0]) and torch.equal(vb[:, :, n], vn[:, :, 0])
    for buf, before in ((kb, k_before), (vb, v_before)):
        assert torch.equal(buf[:, :, :n], before[:, :, :n])
        assert torch.equal(buf[:, :, n + 1:].view(torch.int16), before[:, :, n + 1:].view(torch.int16))


TINY = dict(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_hidden_layers=3,
            num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=8192)


@pytest.fixture(scope="module")
def tiny(gpu):
    from dropkv_amd.e2e_qwen2 import build_model, make_config
    cfg = make_config(**TINY)
    return cfg, build_model(cfg, gpu, dtype=torch.bfloat16, seed=0)


def _prefilled(cfg, model, gpu, L=1024, seed=21):
    from dropkv_amd import hf_cache
    from dropkv_amd.e2e_qwen2 import prefill, random_prompt
    cache = hf_cache.DropKVCache(cfg, keep_ratio=0.1)
    ids = random_prompt(cfg.vocab_size, L, seed=seed, device=gpu)
    return cache, prefill(model, ids, cache)


@pytest.mark.parametrize("use_graph", [False, True])
def test_decoder_matches_eager_transformers_decode(gpu, tiny, use_graph):
    """Same tokens in, the decoder's logits against the eager Transformers
    decode (SDPA over the concatenated compressed cache) at every step."""
    from dropkv_amd.decode import CompressedDecoder
    from dropkv_amd.hf_query import query_capture
    cfg, model = tiny
    cache, tok = _prefilled(cfg, model, gpu)
    dec = CompressedDecoder(model, cache, max_new_tokens=16, use_graph=use_graph)
    g = torch.Generator().manual_seed(5)
    toks = torch.randint(0, cfg.vocab_size, (12, 1, 1), generator=g).to(gpu)
    toks[0] = tok
    with torch.no_grad(), query_capture():
        for t in range(12):
            ref = model(toks[t], past_key_values=cache, use_cache=True, logits_to_keep=1).logits
            got = dec.step(toks[t]).clone()
            torch.testing.assert_close(got.float(), ref.float(), rtol=3e-2, atol=3e-2, msg=f"step {t}")
    assert int(dec.n_rows[0]) == cache.stored_length(0)
    assert int(dec.pos[0, 0]) == cache.get_seq_length()
    # the decoder's buffers hold exactly the rows the eager cache appended
    for i, lay in enumerate(cache.layers):
        n = lay.keys.shape[2]
        torch.testing.assert_close(dec.k_buf[i][:, :, :n].float(), lay.keys.float(), rtol=2e-2, atol=2e-2)


def test_decoder_graph_replays_equal_eager_steps(gpu, tiny):
    """Replays of the captured step, with eager work and synchronisations in
    between, equal the eager decoder on the same inputs bit for bit."""
    from dropkv_amd.decode import CompressedDecoder
    cfg, model = tiny
    cache_a, tok = _prefilled(cfg, model, gpu, seed=22)
    cache_b, _ = _prefilled(cfg, model, gpu, seed=22)
    eager = CompressedDecoder(model, cache_a, max_new_tokens=8, use_graph=False)
    graph = CompressedDecoder(model, cache_b, max_new_tokens=8, use_graph=True)
    for t in range(8):
        a = eager.step(tok).clone()
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=gpu).sum()       # unrelated eager work between replays
        b = graph.step(tok).clone()
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"replay {t}"
        tok = a[:, -1].argmax(-1, keepdim=True)
    with pytest.raises(RuntimeError, match="capacity"):
        graph.step(tok)
