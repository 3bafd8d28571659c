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
