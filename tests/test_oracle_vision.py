"""Pins of the vision-tower oracle (CPU).

The reference's vision tower is models/qwen2_5_vl.py:93-531.  The oracle is
checked against transformers' Qwen2.5-VL vision code (an independent
implementation installed in this image), hand-derived known answers, and
properties of the rotation.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import vision as ov

GRIDS = [[(1, 4, 12)], [(1, 16, 16)], [(1, 18, 30)], [(2, 8, 6)], [(1, 4, 4), (1, 20, 34), (2, 6, 10)],
         [(1, 154, 274)]]


def _hf():
    return pytest.importorskip("transformers.vision_utils")


def test_window_index_known_answer():
    """grid (1, 4, 12), window 56 px, merge 2, patch 14: 2x6 units in windows of 2x2.
    pad_h = 2 - 2 % 2 = 2 adds an empty window row and pad_w = 2 a column; both are
    dropped from the boundaries."""
    idx, cu = ov.window_index([(1, 4, 12)], 56, 2, 14)
    assert idx.tolist() == [0, 1, 6, 7, 2, 3, 8, 9, 4, 5, 10, 11]
    assert cu == [0, 16, 32, 48]


def test_rot_pos_ids_known_answer():
    """(1, 2, 4) with merge 2: two 2x2 blocks, block-major."""
    got = ov.rot_pos_ids(1, 2, 4, 2).tolist()
    assert got == [[0, 0], [0, 1], [1, 0], [1, 1], [0, 2], [0, 3], [1, 2], [1, 3]]
    assert ov.rot_pos_ids(2, 2, 2, 2).tolist() == [[0, 0], [0, 1], [1, 0], [1, 1]] * 2


@pytest.mark.parametrize("grids", GRIDS, ids=lambda g: "+".join("x".join(map(str, x)) for x in g))
def test_layout_matches_transformers(grids):
    vu = _hf()
    g = torch.tensor(grids)
    pos = vu.get_vision_position_ids(g, 2).numpy()
    assert np.array_equal(np.concatenate([ov.rot_pos_ids(t, h, w, 2) for t, h, w in grids]), pos)
    widx, cu = vu.get_vision_window_index(g, spatial_merge_size=2, window_size=112, patch_size=14)
    idx, cu_o = ov.window_index(grids, 112, 2, 14)
    assert np.array_equal(idx, widx.numpy())
    assert cu_o == cu.tolist()
    # Whole-image sequences: the reference makes one per image (t*h*w, models/qwen2_5_vl.py:494-503);
    # transformers one per frame.  They agree for single-frame images.
    if all(t == 1 for t, _, _ in grids):
        assert ov.full_cu_seqlens(grids) == vu.get_vision_cu_seqlens(g).tolist()
    assert ov.full_cu_seqlens([(2, 8, 6)]) == [0, 96]


def test_window_index_is_a_permutation_within_images():
    grids = [(1, 4, 4), (1, 20, 34), (2, 6, 10)]
    idx, cu = ov.window_index(grids, 112, 2, 14)
    assert sorted(idx.tolist()) == list(range(idx.size))
    assert cu[-1] == 4 * idx.size and all(b > a for a, b in zip(cu, cu[1:]))
    assert max(b - a for a, b in zip(cu, cu[1:])) <= 4 * 16     # 4x4 units of 2x2 patches


def _rne_bf16(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (nearest, ties to even) with integer arithmetic."""
    b = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16 << 16
    return b.astype(np.uint32).view(np.float32)


def test_rotary_angles():
    """fp32 angles equal transformers' rotary embedding of the position ids; the
    reference's bf16 angles are those rounded to nearest-even bf16."""
    from transformers.models.qwen2_5_vl.modeling_qwen2_5_vl import Qwen2_5_VisionRotaryEmbedding
    vu = _hf()
    g = torch.tensor([(1, 20, 34)])
    pos = vu.get_vision_position_ids(g, 2)
    rot = Qwen2_5_VisionRotaryEmbedding(40)
    assert torch.equal(ov.inv_freq(80), rot.inv_freq)
    ref = rot(pos)
    a32 = ov.rotary_angles(pos.numpy(), 80, bf16_angles=False)
    assert torch.equal(a32, ref)
    a16 = ov.rotary_angles(pos.numpy(), 80, bf16_angles=True)
    assert np.array_equal(a16.numpy(), _rne_bf16(ref.numpy()))
    assert (a16 != a32).any()   # the rounding is visible at these positions


def test_rope_bf16_against_fp32_rotation():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 4, 80, generator=g).to(torch.bfloat16)
    ang = ov.rotary_angles(ov.rot_pos_ids(1, 8, 8, 2), 80)
    emb = torch.cat((ang, ang), -1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    got = ov.rope_bf16(x, cos, sin).float()
    xf = x.float()
    ref = xf * cos.float()[:, None] + torch.cat((-xf[..., 40:], xf[..., :40]), -1) * sin.float()[:, None]
    # three bf16 roundings: within 2 ulps of the larger term
    ulp = torch.maximum((xf * cos.float()[:, None]).abs(), ref.abs()).clamp_min(1e-30) * 2.0 ** -7
    assert ((got - ref).abs() <= 2 * ulp + 1e-30).all()
    # angle 0: identity, bit for bit
    one, zero = torch.ones(64, 80, dtype=torch.bfloat16), torch.zeros(64, 80, dtype=torch.bfloat16)
    assert torch.equal(ov.rope_bf16(x, one, zero), x)
    # a flipped sign in rotate_half fails the fp32 comparison
    bad = (xf * cos.float()[:, None] + torch.cat((xf[..., 40:], xf[..., :40]), -1) * sin.float()[:, None])
    assert not ((bad - ref).abs() <= 2 * ulp + 1e-30).all()


TINY = dict(depth=3, hidden_size=64, intermediate_size=96, num_heads=4, out_hidden_size=48, patch_size=14,
            spatial_merge_size=2, temporal_patch_size=2, window_size=56, fullatt_block_indexes=[1],
            in_channels=3, hidden_act="silu")


@pytest.mark.parametrize("grids", [[(1, 8, 12)], [(1, 4, 6), (1, 10, 8)], [(2, 4, 4)]],
                         ids=["one", "two", "video"])
def test_forward_matches_transformers(grids):
    """fp32 oracle (fp32 angles) == transformers' vision tower on a tiny config."""
    from transformers.models.qwen2_5_vl.configuration_qwen2_5_vl import Qwen2_5_VLVisionConfig
    from transformers.models.qwen2_5_vl.modeling_qwen2_5_vl import Qwen2_5_VisionTransformerPretrainedModel
    cfg = Qwen2_5_VLVisionConfig(**TINY)
    cfg._attn_implementation = "eager"
    model = Qwen2_5_VisionTransformerPretrainedModel(cfg).float().eval()
    params = ov.random_params(TINY, seed=5)
    missing, unexpected = model.load_state_dict(params, strict=False)
    assert not unexpected and all("inv_freq" in m for m in missing)
    n = sum(t * h * w for t, h, w in grids)
    pix = torch.randn(n, 3 * 2 * 14 * 14, generator=torch.Generator().manual_seed(7))
    got = ov.vision_forward(params, pix, grids, TINY, bf16_angles=False)
    if any(t > 1 for t, _, _ in grids):
        # transformers attends per frame in the whole-image blocks; the reference per image.
        # With no whole-image block the two agree.
        cfg2 = dict(TINY, fullatt_block_indexes=[])
        model.fullatt_block_indexes = []
        got = ov.vision_forward(params, pix, grids, cfg2, bf16_angles=False)
    with torch.no_grad():
        ref = model(pix, torch.tensor(grids)).pooler_output
    assert got.shape == ref.shape == (n // 4, 48)
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)
    # The reference's bf16 angles move the output (slightly, at these small positions).
    q = ov.vision_forward(params, pix, grids, TINY if all(t == 1 for t, _, _ in grids) else cfg2)
    assert (q - got).abs().max() > 1e-6
