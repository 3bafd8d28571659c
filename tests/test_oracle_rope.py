"""Pins the rotary oracle (oracle/rope.py).

Independent checks: transformers' own Qwen2.5-VL rotary embedding and M-RoPE
position code (installed in this image, not part of the reference), a float64
complex-number rotation, the composition law R(a)R(b) = R(a+b), norm
preservation, and hand-derived M-RoPE positions for the 4K-image request.
"""
from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from oracle import rope as orope

hf = pytest.importorskip("transformers.models.qwen2_5_vl.modeling_qwen2_5_vl")
SECTION = [16, 24, 24]


def _hf_rotary():
    from transformers import Qwen2_5_VLConfig

    tc = Qwen2_5_VLConfig().text_config
    assert tc.hidden_size // tc.num_attention_heads == 128
    return hf.Qwen2_5_VLRotaryEmbedding(tc)


def _hf_rotate(k, pos3):
    """transformers' M-RoPE of k [n, H, 128] (fp32) at positions pos3 [3, n]."""
    rot = _hf_rotary()
    pos = torch.as_tensor(pos3)[:, None, :]
    cos, sin = rot(k, pos)
    kk = k.transpose(0, 1)[None]  # [1, H, n, 128]
    _, out = hf.apply_multimodal_rotary_pos_emb(kk, kk, cos, sin, SECTION, unsqueeze_dim=1)
    return out[0].transpose(0, 1)


def test_inv_freq_matches_transformers():
    assert torch.equal(orope.inv_freq(128, 1e6), _hf_rotary().inv_freq.float())


def test_section_of_pair_matches_transformers_layout():
    # Rotate a basis vector with only one section's position nonzero; only that section's pairs move.
    n = 1
    k = torch.randn(n, 1, 128, generator=torch.Generator().manual_seed(0))
    sec = orope.section_of_pair(128, SECTION)
    for s in range(3):
        pos = np.zeros((3, n), dtype=np.int64)
        pos[s] = 37
        out = _hf_rotate(k, pos)
        moved = ~torch.isclose(out, k, atol=1e-6, rtol=0)[0, 0]
        pairs_moved = moved[:64] | moved[64:]
        assert torch.equal(pairs_moved, torch.as_tensor(sec == s)), f"section {s}"


@pytest.mark.parametrize("delta", [(48, 48, 48), (88, 88, 88), (-40, -40, -40), (5, 17, -3), (0, 0, 0)])
def test_rerotation_moves_keys_to_new_position(delta):
    """R(delta) applied to HF-rotated K at p equals HF-rotated K at p + delta (fp32)."""
    g = torch.Generator().manual_seed(1)
    n = 64
    k = torch.randn(n, 2, 128, generator=g)
    p0 = np.stack([np.full(n, 40), 40 + np.arange(n) // 8, 40 + np.arange(n) % 8])
    cached = _hf_rotate(k, p0)
    moved = _hf_rotate(k, p0 + np.asarray(delta)[:, None])
    cs = orope.rerotation_cos_sin([list(delta)], 128, 1e6, SECTION)
    got = orope.rerotate_k(cached, cs)
    assert (got - moved).abs().max().item() < 2e-4


def test_rerotation_matches_complex_float64():
    g = torch.Generator().manual_seed(2)
    k = torch.randn(10, 2, 128, generator=g)
    delta = (7, -13, 29)
    cs = orope.rerotation_cos_sin([list(delta)], 128, 1e6, SECTION)
    got = orope.rerotate_k(k, cs)
    inv = 1.0 / (1e6 ** (np.arange(0, 128, 2) / 128.0))
    d = np.asarray(delta)[orope.section_of_pair(128, SECTION)]
    z = (k[..., :64].double().numpy() + 1j * k[..., 64:].double().numpy()) * np.exp(1j * d * inv)
    ref = np.concatenate([z.real, z.imag], axis=-1)
    assert np.abs(got.double().numpy() - ref).max() < 1e-4


def test_rerotation_composition_inverse_and_norm():
    g = torch.Generator().manual_seed(3)
    k = torch.randn(32, 2, 128, generator=g, dtype=torch.float32)
    a, b = [11, 11, 11], [-4, 30, 2]
    ab = [x + y for x, y in zip(a, b)]
    ra = orope.rerotation_cos_sin([a], 128, 1e6, SECTION)
    rb = orope.rerotation_cos_sin([b], 128, 1e6, SECTION)
    rab = orope.rerotation_cos_sin([ab], 128, 1e6, SECTION)
    two = orope.rerotate_k(orope.rerotate_k(k, ra), rb)
    one = orope.rerotate_k(k, rab)
    assert (two - one).abs().max().item() < 1e-4
    back = orope.rerotate_k(orope.rerotate_k(k, ra), orope.rerotation_cos_sin([[-x for x in a]], 128, 1e6, SECTION))
    assert (back - k).abs().max().item() < 1e-5
    r = orope.rerotate_k(k, rab)
    n0 = k[..., :64] ** 2 + k[..., 64:] ** 2
    n1 = r[..., :64] ** 2 + r[..., 64:] ** 2
    assert torch.allclose(n0, n1, rtol=1e-5, atol=1e-5)


def test_zero_delta_is_bit_identity_in_bf16():
    k = (torch.randn(16, 2, 128, generator=torch.Generator().manual_seed(4))).to(torch.bfloat16)
    k[0, 0, 0] = -0.0  # signed zeros survive
    cs = orope.rerotation_cos_sin([[0, 0, 0]], 128, 1e6, SECTION)
    assert torch.equal(orope.rerotate_k(k, cs).view(torch.int16), k.view(torch.int16))


def test_uniform_delta_reduces_to_reference_1d_cache_row():
    """With dt = dh = dw the table is row delta of the reference's 1-D cos/sin cache.

    The 1-D cache is built as layers/rotary_embedding.py:29-35 does:
    freqs = t (x) inv_freq in fp32, then cos and sin.
    """
    inv = orope.inv_freq(128, 1e6)
    t = torch.arange(200, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv)
    cs = orope.rerotation_cos_sin([[88, 88, 88]], 128, 1e6, SECTION)[0]
    assert torch.equal(cs[:, 0], freqs.cos()[88]) and torch.equal(cs[:, 1], freqs.sin()[88])


def _hf_rope_index(segments):
    """Positions from transformers' get_rope_index for a text/image sequence (images only)."""
    ns = types.SimpleNamespace()
    ns.config = types.SimpleNamespace(vision_config=types.SimpleNamespace(spatial_merge_size=2, tokens_per_second=4))
    ns.get_vision_position_ids = lambda *a, **kw: hf.Qwen2_5_VLModel.get_vision_position_ids(ns, *a, **kw)
    ids, types_, grids = [], [], []
    for kind, val in segments:
        if kind == "text":
            ids += [1] * val
            types_ += [0] * val
        else:
            t, h, w = val
            n = t * (h // 2) * (w // 2)
            ids += [151655] * n
            types_ += [1] * n
            grids.append(list(val))
    pos, _ = hf.Qwen2_5_VLModel.get_rope_index(ns, torch.tensor([ids]), torch.tensor([types_]),
                                               image_grid_thw=torch.tensor(grids))
    return pos[:, 0].numpy()


def test_mrope_positions_match_transformers():
    segs = [("text", 5), ("image", (1, 6, 10)), ("text", 3), ("image", (1, 4, 4)), ("text", 2)]
    ours, starts = orope.mrope_positions(segs)
    assert np.array_equal(ours, _hf_rope_index(segs))
    assert starts == [5, 5 + 5 + 3]


def test_mrope_positions_4k_image_known_answer():
    # 128 text + 3840x2160 image (patch grid 154 x 274 -> 77 x 137 merged) + 64 text
    pos, starts = orope.mrope_positions([("text", 128), ("image", (1, 154, 274)), ("text", 64)])
    img = pos[:, 128:128 + 10549]
    assert starts == [128]
    assert (img[0] == 128).all()
    assert img[1].min() == 128 and img[1].max() == 204
    assert img[2].min() == 128 and img[2].max() == 264
    assert list(pos[0, -64:]) == list(range(265, 329))


# ----------------------------------------------------------------------------- fused RoPE + store oracle
def test_rope_cache_matches_transformers_cos_sin():
    """Row p of the cos/sin cache equals transformers' cos/sin at position p (first half of its 128 channels)."""
    cache = orope.rope_cache(3000, 128, 1e6)[:, 0]
    pos = np.arange(0, 3000, 7)
    cos, sin = _hf_rotary()(torch.zeros(1, 1, 128), torch.as_tensor(np.stack([pos] * 3))[:, None, :])
    assert torch.equal(cache[pos, :64], cos[0, 0, :, :64].float())
    assert torch.equal(cache[pos, 64:], sin[0, 0, :, :64].float())
    assert torch.equal(cos[0, 0, :, :64], cos[0, 0, :, 64:])  # transformers duplicates the half


def test_rope_store_matches_transformers_mrope():
    """fp32 q/k rotated by the oracle at M-RoPE positions == transformers' apply_multimodal_rotary_pos_emb."""
    pos, _ = orope.mrope_positions([("text", 7), ("image", (1, 10, 14)), ("text", 9)])
    n = pos.shape[1]
    g = torch.Generator().manual_seed(30)
    q = torch.randn(n, 4, 128, generator=g)
    k = torch.randn(n, 2, 128, generator=g)
    cache = orope.rope_cache(512, 128, 1e6)
    q_rot, k_rot = orope.rope_store_kvcache(pos, q, k, None, cache, SECTION)
    assert (q_rot - _hf_rotate(q, pos)).abs().max().item() < 1e-5
    assert (k_rot - _hf_rotate(k, pos)).abs().max().item() < 1e-5


def test_rope_store_planted_mistakes_are_caught():
    """A wrong section order or a sign flip in the oracle breaks the transformers comparison."""
    pos = np.stack([np.arange(40), 100 + np.arange(40), 300 + np.arange(40)])
    k = torch.randn(40, 2, 128, generator=torch.Generator().manual_seed(31))
    cache = orope.rope_cache(512, 128, 1e6)
    ref = _hf_rotate(k, pos)
    good, _ = orope.rope_store_kvcache(pos, k, k, None, cache, SECTION)
    assert (good - ref).abs().max().item() < 1e-5
    swapped, _ = orope.rope_store_kvcache(pos, k, k, None, cache, [24, 24, 16])
    assert (swapped - ref).abs().max().item() > 1e-2
    cos, sin = orope.rope_rows(pos, cache, SECTION)
    flipped = orope.apply_rotary_emb(k, cos, -sin)
    assert (flipped - ref).abs().max().item() > 1e-2


def test_rope_store_1d_is_uniform_mrope_and_reference_gather():
    """1-D positions == [3, n] with equal rows; both equal the reference's cache gather + chunk."""
    g = torch.Generator().manual_seed(32)
    q = torch.randn(50, 4, 128, generator=g).to(torch.bfloat16)
    pos = np.random.default_rng(32).integers(0, 1000, 50)
    cache = orope.rope_cache(1000, 128, 1e6)
    a, _ = orope.rope_store_kvcache(pos, q, q, None, cache)
    b, _ = orope.rope_store_kvcache(np.stack([pos] * 3), q, q, None, cache, SECTION)
    cos, sin = cache[torch.as_tensor(pos)].chunk(2, dim=-1)  # layers/rotary_embedding.py:45-47
    x1, x2 = torch.chunk(q.float(), 2, dim=-1)
    c = torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(torch.bfloat16)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(a.view(torch.int16), c.view(torch.int16))


def test_rope_store_scatter_semantics():
    """Stored rows are the rotated k and the raw v; slot -1 and other rows untouched."""
    g = torch.Generator().manual_seed(33)
    n, hkv = 6, 2
    q = torch.randn(n, 4, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(n, hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(n, hkv, 128, generator=g).to(torch.bfloat16)
    kc = torch.randn(2, 8, hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(2, 8, hkv, 128, generator=g).to(torch.bfloat16)
    kc0, vc0 = kc.clone(), vc.clone()
    slots = np.array([3, -1, 0, 15, 8, 9], dtype=np.int32)
    cache = orope.rope_cache(64, 128, 1e6)
    _, k_rot = orope.rope_store_kvcache(np.arange(n) + 5, q, k, v, cache, None, kc, vc, slots)
    fk, fv, fk0, fv0 = kc.view(16, hkv, 128), vc.view(16, hkv, 128), kc0.view(16, hkv, 128), vc0.view(16, hkv, 128)
    for i, s in enumerate(slots):
        if s >= 0:
            assert torch.equal(fk[s].view(torch.int16), k_rot[i].view(torch.int16))
            assert torch.equal(fv[s].view(torch.int16), v[i].view(torch.int16))
    untouched = [r for r in range(16) if r not in set(slots.tolist())]
    assert torch.equal(fk[untouched], fk0[untouched]) and torch.equal(fv[untouched], fv0[untouched])
    assert not torch.equal(k_rot, k)  # positions 5.. rotate


def test_rope_cache_matches_engine_rotary_module():
    from vlcache_amd.layers.rotary_embedding import MRotaryEmbedding

    m = MRotaryEmbedding(128, 128, 2048, 1e6, SECTION)
    assert torch.equal(m.cos_sin_cache, orope.rope_cache(2048, 128, 1e6))


@pytest.mark.parametrize("deltas,section", [
    ([[88, 88, 88]], (16, 24, 24)),
    ([[-5, 3, 7], [48, 48, 48], [0, 0, 0]], (16, 24, 24)),
    ([12, -7], None),
    ([[3, 1, 2]], (8, 12, 12)),
])
def test_engine_rotation_table_is_the_oracle_table(deltas, section):
    """The engine's (cos, sin) table (kernels.rerotation_table, per-model constants cached)
    equals the oracle's bit for bit, before and after the cache is warm."""
    from vlcache_amd import kernels

    hd = 2 * (sum(section) if section else 64)
    want = orope.rerotation_cos_sin(deltas, hd, 1e6, None if section is None else list(section))
    for _ in range(2):
        got = kernels.rerotation_table(deltas, hd, 1e6, None if section is None else list(section))
        assert got.dtype == torch.float32 and torch.equal(got, want)
