"""One Ouro-1.4B attention layer over the hip backend (models/ouro.py:96-112).

The caller's sequence at the model's real sizes (hidden 2048, 16/16 heads,
head_dim 128, bf16): q/k/v projections, RoPE, KV write, paged attention over
mixed-depth LAST-EXITED history, o_proj.  The fused rotary write must give the
same bits as the reference's unfused sequence (rotate, then _write_prepared),
and the attention output must match the CPU oracle on the same pages.
"""

import pytest
import torch

from oracle import rope
from oracle.paged_attention import paged_attention_cpu

pytestmark = pytest.mark.gpu

DEV = "cuda"
HIDDEN, HEADS, D, LAYERS, LOOPS, PAGE = 2048, 16, 128, 2, 4, 16
THETA = 1_000_000.0


def test_ouro_attention_layer_fused_and_unfused_agree():
    from vllm_rlt_amd import KVCacheManager

    g = torch.Generator().manual_seed(21)
    lengths = torch.randint(1, 700, (24,), generator=g).tolist()
    depths = torch.randint(0, LOOPS, (24,), generator=g).tolist()
    blocks = sum(-(-(n + 1) // PAGE) * LOOPS for n in lengths) + 8

    def fresh():
        cache = KVCacheManager(LAYERS, HEADS, D, blocks, PAGE, LOOPS, device=DEV, dtype=torch.bfloat16)
        cache.key_cache.zero_()
        cache.value_cache.zero_()
        for i, n in enumerate(lengths):
            assert cache.allocate(f"r{i}", n + 1)
        return cache

    fused, plain = fresh(), fresh()
    # History: every earlier position of each request at its depth, on both layers.
    for layer in range(LAYERS):
        for i, (n, depth) in enumerate(zip(lengths, depths)):
            k = (torch.randn(n, HEADS, D, generator=g) * 0.5).to(torch.bfloat16)
            v = torch.randn(n, HEADS, D, generator=g).to(torch.bfloat16)
            for cache in (fused, plain):
                cache.write(layer, [f"r{i}"] * n, [depth] * n, list(range(n)), k.to(DEV), v.to(DEV))

    ids = [f"r{i}" for i in range(len(lengths))]
    hidden = (torch.randn(len(ids), HIDDEN, generator=g) * 0.5).to(DEV, torch.bfloat16)
    w = {name: (torch.randn(HIDDEN, HEADS * D, generator=g) * HIDDEN**-0.5).to(DEV, torch.bfloat16) for name in "qkv"}
    w_o = (torch.randn(HEADS * D, HIDDEN, generator=g) * (HEADS * D) ** -0.5).to(DEV, torch.bfloat16)
    cos, sin = rope.rotary_cos_sin(torch.tensor(lengths), D, THETA, torch.bfloat16)
    cos, sin = cos.to(DEV)[:, None], sin.to(DEV)[:, None]

    layer = 1
    outputs = {}
    for cache, fuse in ((fused, True), (plain, False)):
        batch = cache._prepare_batch(ids, depths, lengths)
        shape = (hidden.shape[0], -1, D)
        q = (hidden @ w["q"]).view(shape)
        k = (hidden @ w["k"]).view(shape)
        v = (hidden @ w["v"]).view(shape)
        if fuse:
            q = cache._write_prepared_rotary(layer, batch, q, k, v, (cos, sin))
        else:
            q = q * cos + rope.rotate_half(q) * sin
            k = k * cos + rope.rotate_half(k) * sin
            cache._write_prepared(layer, batch, k, v)
        attended = cache._attend_prepared(layer, batch, q)
        outputs[fuse] = (q, attended, attended.reshape(hidden.shape[0], -1) @ w_o, batch)
    torch.cuda.synchronize()

    q_f, att_f, out_f, batch = outputs[True]
    q_p, att_p, out_p, _ = outputs[False]
    assert torch.equal(q_f, q_p)
    assert torch.equal(fused.key_cache[:, layer], plain.key_cache[:, layer])
    assert torch.equal(fused.value_cache[:, layer], plain.value_cache[:, layer])
    assert torch.equal(att_f, att_p) and torch.equal(out_f, out_p)

    expected = paged_attention_cpu(
        q_f.cpu(), fused.key_cache[:, layer].cpu(), fused.value_cache[:, layer].cpu(),
        batch.block_tables.cpu(), batch.context_lengths.cpu(),
    )
    assert batch.context_lengths.tolist() == [n + 1 for n in lengths]
    torch.testing.assert_close(att_f.cpu().float(), expected.float(), atol=2e-2, rtol=1e-2)
