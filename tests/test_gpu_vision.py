"""GPU parity of the vision tower (models/qwen2_5_vl.py:93-531) against the CPU oracle.

* vlc_vision_rope_pad: bit for bit against the oracle's bf16 rotation (given the
  same cos/sin tables), v copied, padding zero; the device cos/sin tables within
  one bf16 ulp of the oracle's (torch's cos/sin on host and device may round a
  near-tie differently);
* window and whole-image attention of the zero-padded 80-dim heads, through the
  kernel's 128-dim path and its 80-dim path, against the fp32 oracle under the
  per-(row, head) bar, including 96 rows of a 4K image's whole-image attention
  at full size;
* the whole tower against the fp32 oracle (with the reference's bf16 angles) on
  a tiny configuration and on the public 32-block configuration with small
  images; the bf16 product and the fp32 oracle differ by bf16 rounding through
  the blocks, so the bar is a per-row cosine (stated in each test);
* the engine: a cold request runs the tower and fills the encoder cache, a warm
  request reads it back and reports no vision time.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oattn
from oracle import vision as ov
from tests._util import assert_attn_close, row_cosines, say
from vlcache_amd import kernels
from vlcache_amd.vision import VisionLayout, VisionTransformer, vision_config

pytestmark = pytest.mark.gpu

REAL = dict(depth=32, hidden_size=1280, intermediate_size=3420, num_heads=16, out_hidden_size=2048, patch_size=14,
            spatial_merge_size=2, temporal_patch_size=2, window_size=112, fullatt_block_indexes=[7, 15, 23, 31],
            in_channels=3, hidden_act="silu")
TINY = dict(REAL, depth=3, hidden_size=64, intermediate_size=96, num_heads=4, out_hidden_size=48,
            fullatt_block_indexes=[1])


def _tower(cfg: dict, params: dict, dev) -> VisionTransformer:
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            vt = VisionTransformer(vision_config(cfg, cfg["out_hidden_size"]))
    finally:
        torch.set_default_dtype(prev)
    vt.load_checkpoint_weights({k: v.to(torch.bfloat16) for k, v in params.items()})
    return vt.eval()


def _pixels(grids, seed):
    n = sum(t * h * w for t, h, w in grids)
    return torch.randn(n, 3 * 2 * 14 * 14, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)


def _rope_inputs(dev, grids, heads=16, hd=80, seed=0):
    lay = VisionLayout(grids, 112, 2, 14)
    n = lay.num_patches
    qkv = (torch.randn(n, 3 * heads * hd, generator=torch.Generator().manual_seed(seed))).to(torch.bfloat16)
    with torch.device(dev):
        vt = VisionTransformer(vision_config(dict(TINY, hidden_size=heads * hd, num_heads=heads), 48))
    cos, sin = vt.rope_tables(lay.max_pos)
    return lay, qkv, cos, sin


def test_rope_tables_match_oracle(dev):
    say("vision: bf16 cos/sin tables for positions 0..273")
    _, _, cos, sin = _rope_inputs(dev, [(1, 154, 274)])
    pos = np.stack([np.arange(274), np.zeros(274, np.int64)], -1)
    ang = ov.rotary_angles(pos, 80, bf16_angles=True)[:, :20]
    for got, ref in ((cos, ang.cos()), (sin, ang.sin())):
        ref16 = ref.to(torch.bfloat16)
        diff = (got.cpu().view(torch.int16).int() - ref16.view(torch.int16).int()).abs()
        assert int(diff.max()) <= 1, "cos/sin tables differ by more than one bf16 ulp"


@pytest.mark.parametrize("grids", [[(1, 16, 16)], [(1, 4, 4), (1, 20, 34), (2, 6, 10)], [(1, 154, 274)]],
                         ids=["16x16", "three", "4k"])
def test_vision_rope_pad_bit_exact(dev, grids):
    say(f"vision: vlc_vision_rope_pad grids={grids}")
    lay, qkv, cos, sin = _rope_inputs(dev, grids, seed=len(grids))
    out = kernels.vision_rope_pad(qkv.to(dev), torch.from_numpy(lay.pos_hw).to(dev), cos, sin, 16, 80)
    torch.cuda.synchronize()
    out = out.cpu()
    n = lay.num_patches
    # The oracle's rotation with cos/sin per token gathered from the same tables.
    ph, pw = torch.from_numpy(lay.pos_hw[:, 0]).long(), torch.from_numpy(lay.pos_hw[:, 1]).long()
    c, s = cos.cpu(), sin.cpu()
    c40, s40 = torch.cat((c[ph], c[pw]), -1), torch.cat((s[ph], s[pw]), -1)
    c80, s80 = torch.cat((c40, c40), -1), torch.cat((s40, s40), -1)
    q, k, v = qkv.reshape(n, 3, 16, 80).unbind(1)
    for part, ref in ((0, ov.rope_bf16(q, c80, s80)), (1, ov.rope_bf16(k, c80, s80)), (2, v)):
        assert torch.equal(out[:, part, :, :80].view(torch.int16), ref.view(torch.int16)), f"part {part}"
    assert not out[:, :, :, 80:].view(torch.int16).any(), "padding must be zero"


def test_vision_rope_pad_refuses_bad_tables(dev):
    lay, qkv, cos, sin = _rope_inputs(dev, [(1, 16, 16)])
    with pytest.raises(ValueError):
        kernels.vision_rope_pad(qkv.to(dev), torch.from_numpy(lay.pos_hw).to(dev), cos[:, :10].contiguous(),
                                sin[:, :10].contiguous(), 16, 80)


@pytest.mark.parametrize("hd", [128, 80], ids=["as-128", "hd80"])
@pytest.mark.parametrize("full", [False, True], ids=["windows", "whole-image"])
def test_padded_attention(dev, full, hd):
    """80-dim heads in 128-element rows, through the kernel's 128-dim path (zero dims take
    part in the products) and its 80-dim path (the products skip them)."""
    grids = [(1, 4, 4), (1, 20, 34), (2, 6, 10)]
    say(f"vision: padded 80-dim attention, full={full}, kernel head_dim={hd}, grids={grids}")
    lay, qkv, cos, sin = _rope_inputs(dev, grids, seed=7)
    heads = kernels.vision_rope_pad(qkv.to(dev), torch.from_numpy(lay.pos_hw).to(dev), cos, sin, 16, 80)
    cu = lay.cu_full if full else lay.cu_window
    plan = kernels.plan_attention(cu, cu, 16, 16, hd, False, dev)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    o = kernels.varlen_attention(heads[:, 0], heads[:, 1], heads[:, 2], cu_t, cu_t, 80 ** -0.5, causal=False,
                                 plan=plan, head_dim=hd).cpu()
    hc = heads.cpu()
    ref = oattn.varlen_attention(hc[:, 0, :, :80], hc[:, 1, :, :80], hc[:, 2, :, :80], cu, cu, 80 ** -0.5, False)
    assert_attn_close(o[..., :80], ref, what="padded vision attention")
    assert not o[..., 80:].view(torch.int16).any()


@pytest.mark.parametrize("hd", [128, 80], ids=["as-128", "hd80"])
def test_whole_image_attention_4k_sampled_rows(dev, hd):
    """Whole-image attention over a 4K image's 42196 patches at full size; 96 query rows
    (spread over the sequence, both ends included) against the fp32 oracle."""
    grids = [(1, 154, 274)]
    say(f"vision: 4K whole-image attention, 42196 x 42196, non-causal, kernel head_dim={hd}")
    lay, qkv, cos, sin = _rope_inputs(dev, grids, seed=11)
    heads = kernels.vision_rope_pad(qkv.to(dev), torch.from_numpy(lay.pos_hw).to(dev), cos, sin, 16, 80)
    cu = lay.cu_full
    plan = kernels.plan_attention(cu, cu, 16, 16, hd, False, dev)
    print(f"plan: items={plan.num_items} combines={plan.num_combine}", flush=True)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    o = kernels.varlen_attention(heads[:, 0], heads[:, 1], heads[:, 2], cu_t, cu_t, 80 ** -0.5, causal=False,
                                 plan=plan, head_dim=hd).cpu()
    hc = heads.cpu()
    n = lay.num_patches
    rows = torch.unique(torch.cat([torch.tensor([0, 1, n - 2, n - 1]), torch.linspace(0, n - 1, 92).long()]))
    q = hc[rows, 0, :, :80].float()
    k, v = hc[:, 1, :, :80].float(), hc[:, 2, :, :80].float()
    s = torch.einsum("rhd,nhd->hrn", q, k) * 80 ** -0.5
    ref = torch.einsum("hrn,nhd->rhd", torch.softmax(s, dim=-1), v)
    assert_attn_close(o[rows, :, :80], ref, what="4K whole-image attention rows")
    assert np.isfinite(o.float().numpy()).all()


def test_hd80_refuses_paged_calls_and_foreign_plans(dev):
    lay, qkv, cos, sin = _rope_inputs(dev, [(1, 16, 16)])
    heads = kernels.vision_rope_pad(qkv.to(dev), torch.from_numpy(lay.pos_hw).to(dev), cos, sin, 16, 80)
    cu = lay.cu_window
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    plan128 = kernels.plan_attention(cu, cu, 16, 16, 128, False, dev)
    with pytest.raises(ValueError, match="head_dim"):
        kernels.varlen_attention(heads[:, 0], heads[:, 1], heads[:, 2], cu_t, cu_t, 0.1, causal=False,
                                 plan=plan128, head_dim=80)
    cache = torch.zeros(4, 256, 16, 128, dtype=torch.bfloat16, device=dev)
    bt = torch.zeros(len(cu) - 1, 1, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="head_dim"):
        kernels.varlen_attention(heads[:, 0], cache, cache, cu_t, cu_t, 0.1, causal=False, block_table=bt,
                                 head_dim=80)


def _tower_check(dev, cfg, grids, seed, row_cos_min):
    params = ov.random_params(cfg, seed=seed)
    pix = _pixels(grids, seed + 1)
    vt = _tower(cfg, params, dev)
    got = vt(pix.to(dev), grids).float().cpu()
    ref = ov.vision_forward(params, pix.float(), grids, cfg, bf16_angles=True)
    cos, _, _ = row_cosines(got, ref)
    worst = float(cos.min())
    rel = float((got - ref).norm() / ref.norm())
    print(f"rows={got.shape[0]} worst row cosine {worst:.6f}, relative L2 error {rel:.2e}", flush=True)
    assert got.shape == ref.shape
    assert worst >= row_cos_min, f"worst row cosine {worst:.6f} < {row_cos_min}"
    return vt, pix, got


def test_tower_tiny_config(dev):
    """3 blocks (one whole-image), hidden 64, 4 heads of 16 dims; bar: every output row's
    cosine with the fp32 oracle >= 0.9995."""
    grids = [(1, 8, 12), (1, 4, 6), (1, 18, 30)]
    say(f"vision tower, tiny config, grids={grids}")
    _tower_check(dev, TINY, grids, 3, 0.9995)


def test_tower_public_config_small_images(dev):
    """The public configuration (32 blocks of hidden 1280, 16 heads of 80 dims, whole-image
    attention at blocks 7/15/23/31) on two small images; bar: every output row's cosine
    with the fp32 oracle >= 0.999 (bf16 activations and weights through 32 blocks)."""
    grids = [(1, 16, 16), (1, 20, 34)]
    say(f"vision tower, public config, grids={grids}")
    _tower_check(dev, REAL, grids, 5, 0.999)


def test_tower_two_frame_video(dev):
    """A two-frame grid (t = 2): frames share the patch positions, windows are per frame,
    the whole-image blocks attend over both frames (the reference's one sequence per
    image, models/qwen2_5_vl.py:494-503); bar: per-row cosine >= 0.9995 against the
    fp32 oracle."""
    grids = [(2, 8, 12), (1, 4, 6)]
    say(f"vision tower, tiny config, video grid {grids}")
    _tower_check(dev, TINY, grids, 13, 0.9995)


def test_tower_batch_equals_single_images(dev):
    """Images batched into one call give each image's own embeddings (windows and whole-image
    sequences never cross images); GEMMs may round differently at another row count, so
    the bar is the per-row cosine >= 0.9999."""
    grids = [(1, 8, 12), (1, 18, 30)]
    say("vision tower: batch of two == each alone")
    params = ov.random_params(TINY, seed=9)
    vt = _tower(TINY, params, dev)
    pix = _pixels(grids, 10).to(dev)
    both = vt(pix, grids).float().cpu()
    a = vt(pix[:96], grids[:1]).float().cpu()
    b = vt(pix[96:], grids[1:]).float().cpu()
    cos, _, _ = row_cosines(both, torch.cat([a, b]))
    assert float(cos.min()) >= 0.9999


def test_engine_runs_the_tower_on_a_cold_image(dev):
    """Cold request: the tower runs (vit_time > 0) and its embeddings enter the encoder
    cache; they equal a direct call of the tower bit for bit.  Warm request with the
    same image: a cache hit, no vision time."""
    from vlcache_amd import LLM, SamplingParams

    text = dict(architectures=["Qwen2_5_VLForConditionalGeneration"], hidden_size=256, intermediate_size=512,
                num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1, head_dim=128,
                vocab_size=151936, rms_norm_eps=1e-6, rope_theta=1e6,
                rope_scaling={"type": "mrope", "mrope_section": [16, 24, 24]}, max_position_embeddings=8192,
                tie_word_embeddings=True, image_token_id=151655, eos_token_id=151645,
                vision_config=dict(TINY, out_hidden_size=256))
    say("engine with a vision tower: cold then warm request")
    llm = LLM(text, recompute_ratio=0.1, num_kvcache_blocks=16, max_model_len=4096, enforce_eager=True)
    grid = (1, 20, 34)
    n_img = 10 * 17
    pix = _pixels([grid], 21)
    rng = np.random.default_rng(0)
    toks = lambda p, s: ([int(x) for x in rng.integers(1, 150000, p)] + [151655] * n_img +  # noqa: E731
                         [int(x) for x in rng.integers(1, 150000, s)])
    mm = {"pixel_values": pix, "image_grid_thw": torch.tensor([list(grid)])}
    sp = SamplingParams(temperature=0.6, max_tokens=1)
    cold = llm.generate([toks(40, 16)], sp, mm_inputs=[mm])[0]
    runner = llm.model_runner
    cache = runner.encoder_cache
    assert len(cache) == 1 and cold["vit_time"] > 0
    h = next(iter(cache._entries))
    direct = runner.model.visual(pix.to(dev), [grid])
    assert torch.equal(cache.get(h).view(torch.int16), direct.view(torch.int16))
    warm = llm.generate([toks(128, 16)], sp, mm_inputs=[mm])[0]
    assert warm["vit_time"] == 0.0 and cache.hits >= 2
    # Two cold images in one request, one of them repeated by a second request in the same
    # batch: one tower call over the distinct images; each image's rows equal a direct call.
    g2 = (1, 8, 12)
    pix2 = _pixels([g2], 22)
    toks2 = ([int(x) for x in rng.integers(1, 150000, 20)] + [151655] * (4 * 6) +
             [int(x) for x in rng.integers(1, 150000, 10)] + [151655] * n_img)
    pix3 = _pixels([grid], 23)
    mm2 = {"pixel_values": torch.cat([pix2, pix3]), "image_grid_thw": torch.tensor([list(g2), list(grid)])}
    toks3 = [int(x) for x in rng.integers(1, 150000, 30)] + [151655] * (4 * 6) + [7]
    mm3 = {"pixel_values": pix2, "image_grid_thw": torch.tensor([list(g2)])}
    before = len(cache)
    outs = llm.generate([toks2, toks3], sp, mm_inputs=[mm2, mm3])
    assert all(o["vit_time"] > 0 for o in outs) and len(cache) == before + 2
    keys = list(cache._entries)[-2:]
    for key, (pv, g) in zip(keys, ((pix2, g2), (pix3, grid))):
        direct = runner.model.visual(pv.to(dev), [g])
        assert torch.equal(cache.get(key).view(torch.int16), direct.view(torch.int16))


@pytest.mark.parametrize("seed", range(4))
def test_random_grids(dev, seed):
    """Seeded random batches of 1-3 images (t 1-2, h and w even, 2..60 patches a side):
    the window layout equals the oracle's, the rotary kernel is bit-exact, and the
    80-dim window and whole-image attention pass the per-(row, head) bar."""
    rng = np.random.default_rng(200 + seed)
    grids = [(int(rng.integers(1, 3)), 2 * int(rng.integers(1, 31)), 2 * int(rng.integers(1, 31)))
             for _ in range(int(rng.integers(1, 4)))]
    say(f"vision random grids seed {seed}: {grids}")
    lay, qkv, cos, sin = _rope_inputs(dev, grids, seed=300 + seed)
    idx, cu = ov.window_index(grids, 112, 2, 14)
    assert np.array_equal(lay.window_index, idx) and lay.cu_window == cu
    assert lay.cu_full == ov.full_cu_seqlens(grids)
    heads = kernels.vision_rope_pad(qkv.to(dev), torch.from_numpy(lay.pos_hw).to(dev), cos, sin, 16, 80)
    hc = heads.cpu()
    n = lay.num_patches
    ph, pw = torch.from_numpy(lay.pos_hw[:, 0]).long(), torch.from_numpy(lay.pos_hw[:, 1]).long()
    c, s = cos.cpu(), sin.cpu()
    c80 = torch.cat((c[ph], c[pw], c[ph], c[pw]), -1)
    s80 = torch.cat((s[ph], s[pw], s[ph], s[pw]), -1)
    q, k, v = qkv.reshape(n, 3, 16, 80).unbind(1)
    assert torch.equal(hc[:, 0, :, :80].view(torch.int16), ov.rope_bf16(q, c80, s80).view(torch.int16))
    assert torch.equal(hc[:, 1, :, :80].view(torch.int16), ov.rope_bf16(k, c80, s80).view(torch.int16))
    assert torch.equal(hc[:, 2, :, :80].view(torch.int16), v.view(torch.int16))
    for cu_h in (lay.cu_window, lay.cu_full):
        plan = kernels.plan_attention(cu_h, cu_h, 16, 16, 80, False, dev)
        cu_t = torch.tensor(cu_h, dtype=torch.int32, device=dev)
        o = kernels.varlen_attention(heads[:, 0], heads[:, 1], heads[:, 2], cu_t, cu_t, 80 ** -0.5, causal=False,
                                     plan=plan, head_dim=80).cpu()
        ref = oattn.varlen_attention(hc[:, 0, :, :80], hc[:, 1, :, :80], hc[:, 2, :, :80], cu_h, cu_h,
                                     80 ** -0.5, False)
        assert_attn_close(o[..., :80], ref, what=f"random grids {grids}")
