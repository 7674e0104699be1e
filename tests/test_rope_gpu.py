"""Fused rotary embedding + KV append (rlt_rope_kv_append) against the oracle (GPU).

The rotated q and the written pages must be bit-identical to the unfused
sequence of the reference: q * cos + rotate_half(q) * sin and the same for k
(vllm_rlt/models/ouro.py:104-109), then the index_put append
(vllm_rlt/core/kv_cache_manager.py:531-532).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import rope

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "rotary_cpu.npz"
DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}
BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}


def bits(t):
    return t.contiguous().view(BITS[t.dtype]).cpu()


def random_bits(shape, dtype, seed):
    """Arbitrary finite-or-not bit patterns (pages must stay untouched bitwise)."""
    g = torch.Generator().manual_seed(seed)
    info = torch.iinfo(BITS[dtype])
    return torch.randint(info.min, info.max, shape, generator=g, dtype=torch.int64).to(BITS[dtype]).view(dtype)


@pytest.mark.parametrize("name", ["bf16_ouro", "fp16_ouro", "fp32_ouro", "bf16_tiny"])
def test_reference_golden_bits(name):
    """The reference's own rotation outputs come back bit for bit, in q_out and in the pages."""
    from vllm_rlt_amd import ops

    data = np.load(GOLDEN)
    dtype = DTYPES[str(data[f"{name}/dtype"])]
    x, cos, sin, out = (torch.from_numpy(data[f"{name}/{f}"]).view(dtype) for f in ("x", "cos", "sin", "out"))
    n, heads, d = x.shape
    kc = random_bits((n + 3, 2, 1, heads, d), dtype, 1).cuda()
    vc = random_bits((n + 3, 2, 1, heads, d), dtype, 2).cuda()
    v = random_bits((n, heads, d), dtype, 3)
    blocks = torch.randperm(n + 3, generator=torch.Generator().manual_seed(4))[:n].cuda()
    offsets = torch.zeros(n, dtype=torch.int64, device="cuda")
    q_out = ops.rope_kv_append(kc, vc, 1, blocks, offsets, x.cuda(), x.cuda(), v.cuda(), cos.cuda(), sin.cuda())
    torch.cuda.synchronize()
    assert torch.equal(bits(q_out), bits(out))
    assert torch.equal(bits(kc[blocks, 1, 0]), bits(out))
    assert torch.equal(bits(vc[blocks, 1, 0]), bits(v))


def ouro_case(dtype, rows, hq, hkv, d, seed, page=16, layers=3):
    g = torch.Generator().manual_seed(seed)
    nb = rows + 5
    kc = random_bits((nb, layers, page, hkv, d), dtype, seed + 1)
    vc = random_bits((nb, layers, page, hkv, d), dtype, seed + 2)
    q = (torch.randn(rows, hq, d, generator=g) * 2).to(dtype)
    k = (torch.randn(rows, hkv, d, generator=g) * 2).to(dtype)
    v = random_bits((rows, hkv, d), dtype, seed + 3)
    positions = torch.randint(0, 70000, (rows,), generator=g)
    cos, sin = rope.rotary_cos_sin(positions, d, 1_000_000.0, dtype)
    slots = torch.randperm(nb * page, generator=g)[:rows]
    return kc, vc, q, k, v, cos, sin, slots // page, slots % page


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hq,hkv,d", [(16, 16, 128), (8, 2, 64), (4, 4, 6)])
def test_matches_oracle_bitwise(dtype, hq, hkv, d):
    """Ouro shape, GQA and an odd half-width (scalar path); padding rows are not written."""
    from vllm_rlt_amd import ops

    rows = 37
    kc, vc, q, k, v, cos, sin, blocks, offsets = ouro_case(dtype, rows, hq, hkv, d, seed=hq * d)
    n_write = rows - 4
    exp_k, exp_v = kc.clone(), vc.clone()
    exp_q = rope.rope_append(exp_k, exp_v, 2, blocks, offsets, q, k, v, cos, sin, n_rows=n_write)
    gk, gv = kc.cuda(), vc.cuda()
    got_q = ops.rope_kv_append(
        gk, gv, 2, blocks.cuda(), offsets.cuda(), q.cuda(), k.cuda(), v.cuda(), cos.cuda(), sin.cuda(), n_rows=n_write
    )
    torch.cuda.synchronize()
    assert torch.equal(bits(got_q), bits(exp_q))
    assert torch.equal(bits(gk), bits(exp_k))
    assert torch.equal(bits(gv), bits(exp_v))


def test_strided_views_and_in_place_q():
    """Head-major q/k views, the model's [batch, 1, D] cos/sin, and q rotated in place."""
    from vllm_rlt_amd import ops

    dtype, rows, hq, hkv, d = torch.bfloat16, 19, 16, 16, 128
    kc, vc, q, k, v, cos, sin, blocks, offsets = ouro_case(dtype, rows, hq, hkv, d, seed=7)
    exp_k, exp_v = kc.clone(), vc.clone()
    exp_q = rope.rope_append(exp_k, exp_v, 0, blocks, offsets, q, k, v, cos, sin)
    gq = q.transpose(0, 1).contiguous().cuda().transpose(0, 1)  # [rows, hq, d] view, head stride rows*d
    gk = k.transpose(0, 1).contiguous().cuda().transpose(0, 1)
    kcg, vcg = kc.cuda(), vc.cuda()
    out = ops.rope_kv_append(
        kcg, vcg, 0, blocks.cuda(), offsets.cuda(), gq, gk, v.cuda(), cos.cuda()[:, None], sin.cuda()[:, None], out=gq
    )
    torch.cuda.synchronize()
    assert out.data_ptr() == gq.data_ptr()
    assert torch.equal(bits(gq), bits(exp_q))
    assert torch.equal(bits(kcg), bits(exp_k)) and torch.equal(bits(vcg), bits(exp_v))


def test_out_of_range_addresses_are_skipped_but_q_is_rotated():
    from vllm_rlt_amd import ops

    dtype, rows = torch.bfloat16, 4
    kc, vc, q, k, v, cos, sin, blocks, offsets = ouro_case(dtype, rows, 16, 16, 128, seed=11)
    blocks[1] = kc.shape[0]  # one past the pool
    offsets[2] = 16  # one past the page
    before_k, before_v = bits(kc), bits(vc)
    kcg, vcg = kc.cuda(), vc.cuda()
    out = ops.rope_kv_append(kcg, vcg, 1, blocks.cuda(), offsets.cuda(), q.cuda(), k.cuda(), v.cuda(), cos.cuda(), sin.cuda())
    torch.cuda.synchronize()
    assert torch.equal(bits(out), bits(rope.apply_rotary(q, cos, sin)))
    exp_k, exp_v = kc.clone(), vc.clone()
    keep = [0, 3]
    rope.rope_append(exp_k, exp_v, 1, blocks[keep], offsets[keep], q[keep], k[keep], v[keep], cos[keep], sin[keep])
    assert torch.equal(bits(kcg), bits(exp_k)) and torch.equal(bits(vcg), bits(exp_v))
    assert not torch.equal(bits(kcg), before_k) and not torch.equal(bits(vcg), before_v)


def test_manager_rotary_write_equals_rotation_then_write():
    """_write_prepared_rotary == rotate (models/ouro.py:108-109) + _write_prepared, then attention agrees."""
    from vllm_rlt_amd import KVCacheManager

    def fresh():
        return KVCacheManager(
            num_layers=2, num_kv_heads=4, head_dim=64, num_blocks=24, block_size=16, max_loops=4, device="cuda",
            dtype=torch.bfloat16,
        )

    fused, plain = fresh(), fresh()
    for cache in (fused, plain):
        assert cache.allocate("a", 40) and cache.allocate("b", 40)
        cache.key_cache.zero_()
        cache.value_cache.zero_()
    g = torch.Generator().manual_seed(3)
    rows = [("a", 0, p) for p in range(20)] + [("b", 2, p) for p in range(7)]
    ids, depths, positions = zip(*rows)
    n = len(rows)
    q = (torch.randn(n, 8, 64, generator=g)).to(torch.bfloat16).cuda()
    k = (torch.randn(n, 4, 64, generator=g)).to(torch.bfloat16).cuda()
    v = (torch.randn(n, 4, 64, generator=g)).to(torch.bfloat16).cuda()
    cos, sin = rope.rotary_cos_sin(torch.tensor(positions), 64, 1_000_000.0, torch.bfloat16)
    emb = (cos.cuda()[:, None], sin.cuda()[:, None])
    outs = []
    for cache, fuse in ((fused, True), (plain, False)):
        batch = cache._prepare_batch(list(ids), list(depths), list(positions))
        if fuse:
            q_rot = cache._write_prepared_rotary(1, batch, q, k, v, emb)
        else:
            q_rot = q * emb[0] + rope.rotate_half(q) * emb[1]
            cache._write_prepared(1, batch, k * emb[0] + rope.rotate_half(k) * emb[1], v)
        outs.append((q_rot, cache._attend_prepared(1, batch, q_rot)))
    torch.cuda.synchronize()
    assert torch.equal(bits(fused.key_cache), bits(plain.key_cache))
    assert torch.equal(bits(fused.value_cache), bits(plain.value_cache))
    assert torch.equal(bits(outs[0][0]), bits(outs[1][0]))
    assert torch.equal(bits(outs[0][1]), bits(outs[1][1]))
