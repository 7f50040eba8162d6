"""CPU tests of the drop-in layer: duck typing, patch counts, copied state, Swin window
geometry and masks, and the toy-encoder pairs (no kernel launches)."""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn

import elsa_amd
from elsa_amd.timm_dropin import ElsaTimmSwinWindowAttention, ElsaTimmVitAttention
from elsa_amd.timm_dropin_bwd import ElsaTrainTimmSwinWindowAttention, ElsaTrainTimmVitAttention
from elsa_amd.vision_models import (SwinTransformerBlock, relative_position_index, swin_tiny_patch4_window7,
                                    vit_tiny_patch16)


def test_vit_tiny_patch_counts_and_state():
    torch.manual_seed(0)
    m = vit_tiny_patch16(224)
    ref_qkv = m.blocks[3].attn.qkv.weight.detach().clone()
    rep = elsa_amd.patch_timm_attention(m)
    assert rep == elsa_amd.PatchReport(vit_attention=12, swin_window_attention=0) and rep.total == 12
    a = m.blocks[3].attn
    assert isinstance(a, ElsaTimmVitAttention) and a.num_heads == 3 and a.head_dim == 64 and a.attn_dim == 192
    assert torch.equal(a.qkv.weight, ref_qkv)


def test_swin_tiny_patch_counts_train():
    m = swin_tiny_patch4_window7(224)
    rep = elsa_amd.patch_timm_attention_train(m)
    assert rep == elsa_amd.TrainPatchReport(vit_attention=0, swin_window_attention=12)
    assert isinstance(m.layers[2].blocks[5].attn, ElsaTrainTimmSwinWindowAttention)
    assert m.layers[2].blocks[5].attn.head_dim == 32


def test_patch_rejects_models_without_attention():
    with pytest.raises(ValueError, match="no compatible timm"):
        elsa_amd.patch_timm_attention(nn.Sequential(nn.Linear(4, 4)))
    with pytest.raises(ValueError, match="no compatible timm"):
        elsa_amd.patch_timm_attention_train(nn.Sequential(nn.Linear(4, 4)))


def test_swin_v2_style_module_is_not_patched():
    m = swin_tiny_patch4_window7(224)
    m.layers[0].blocks[0].attn.logit_scale = nn.Parameter(torch.zeros(3, 1, 1))
    rep = elsa_amd.patch_timm_attention(m)
    assert rep.swin_window_attention == 11


def test_vit_dropin_rejects_mask_and_dropout():
    m = vit_tiny_patch16(224)
    elsa_amd.patch_timm_attention(m)
    with pytest.raises(ValueError, match="unmasked"):
        m.blocks[0].attn(torch.zeros(1, 197, 192), attn_mask=torch.zeros(197, 197))
    t = vit_tiny_patch16(224)
    t.blocks[0].attn.attn_drop.p = 0.1
    elsa_amd.patch_timm_attention_train(t)
    t.train()
    with pytest.raises(ValueError, match="dropout"):
        t.blocks[0].attn(torch.zeros(1, 197, 192))


def test_relative_position_index_closed_form():
    idx = relative_position_index(2, 3)
    # (dy + 1) * 5 + (dx + 2) for query (y1,x1), key (y2,x2), dy = y1 - y2, dx = x1 - x2
    coords = [(y, x) for y in range(2) for x in range(3)]
    for i, (y1, x1) in enumerate(coords):
        for j, (y2, x2) in enumerate(coords):
            assert idx[i, j] == (y1 - y2 + 1) * 5 + (x1 - x2 + 2)


def test_shifted_window_mask_values():
    blk = SwinTransformerBlock(96, (14, 14), 3, 7, shift=True)
    assert blk.shift_size == (3, 3)
    mask = blk.attn_mask
    assert mask.shape == (4, 49, 49)
    assert set(mask.unique().tolist()) == {0.0, -100.0}
    assert torch.all(mask[0] == 0)  # top-left window is not split by the shift
    no_shift = SwinTransformerBlock(96, (7, 7), 3, 7, shift=True)
    assert no_shift.shift_size == (0, 0) and no_shift.attn_mask is None


def test_set_window_size_resizes_table_and_index():
    m = swin_tiny_patch4_window7(224)
    elsa_amd.patch_timm_attention(m)
    a = m.layers[0].blocks[0].attn
    assert isinstance(a, ElsaTimmSwinWindowAttention)
    a.set_window_size(8)
    assert a.window_size == (8, 8) and a.window_area == 64
    assert a.relative_position_bias_table.shape == (15 * 15, 3)
    assert a.relative_position_index.shape == (64, 64) and int(a.relative_position_index.max()) == 15 * 15 - 1


def test_model_pairs_share_weights():
    base, elsa = elsa_amd.make_model_pair(dim=96, depth=2, heads=3)
    for (n1, p1), (n2, p2) in zip(base.state_dict().items(), elsa.state_dict().items()):
        assert n1 == n2 and torch.equal(p1, p2)
    assert all(layer.core.backend == "sdpa" for layer in base.layers)
    assert all(layer.core.backend == "elsa" for layer in elsa.layers)
    assert base.layers[0].qkv.weight.data_ptr() != elsa.layers[0].qkv.weight.data_ptr()  # copies, not aliases
    tb, te = elsa_amd.make_train_model_pair(dim=96, depth=1, heads=3, is_causal=True)
    assert isinstance(te, elsa_amd.TrainableTransformerEncoder) and te.layers[0].core.trainable
    assert te.layers[0].core.is_causal and te.layers[0].core.elsa_kwargs["algorithm"] == "paper_scan"
    x = torch.randn(1, 16, 96)
    assert base(x).shape == (1, 16, 96) and tb(x).shape == (1, 16, 96)
    with pytest.raises(ValueError, match="divisible"):
        elsa_amd.make_model_pair(dim=95, heads=3)
    with pytest.raises(ValueError, match="backend"):
        elsa_amd.TransformerEncoder(dim=96, heads=3, backend="flash")
    with pytest.raises(ValueError, match="SDPA kind"):
        elsa_amd.TransformerEncoder(dim=96, heads=3, backend="sdpa", sdpa_kind="fast")


def test_encoder_layer_is_the_pre_norm_block():
    """The SDPA baseline against the same block written out with plain torch ops."""
    torch.manual_seed(4)
    base, _ = elsa_amd.make_model_pair(dim=48, depth=2, heads=3, mlp_ratio=2.0, is_causal=True)
    x = torch.randn(2, 10, 48)
    want = x
    for layer in base.layers:
        h = torch.nn.functional.layer_norm(want, (48,), layer.norm1.weight, layer.norm1.bias)
        qkv = h @ layer.qkv.weight.T + layer.qkv.bias
        q, k, v = (t.reshape(2, 10, 3, 16).transpose(1, 2) for t in qkv.split(48, dim=-1))
        s = (q @ k.transpose(-1, -2)) / 4.0 + torch.triu(torch.full((10, 10), float("-inf")), 1)
        a = (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(2, 10, 48)
        want = want + a @ layer.proj.weight.T + layer.proj.bias
        h = torch.nn.functional.layer_norm(want, (48,), layer.norm2.weight, layer.norm2.bias)
        h = torch.nn.functional.gelu(h @ layer.fc1.weight.T + layer.fc1.bias)
        want = want + h @ layer.fc2.weight.T + layer.fc2.bias
    want = torch.nn.functional.layer_norm(want, (48,), base.norm.weight, base.norm.bias)
    torch.testing.assert_close(base(x), want, atol=1e-5, rtol=1e-5)


def test_inference_encoder_refuses_gradients_through_elsa():
    _, elsa = elsa_amd.make_model_pair(dim=48, depth=1, heads=3)
    qkv = torch.zeros(1, 4, 3, 3, 16, requires_grad=True)
    with pytest.raises(RuntimeError, match="inference-only"):
        elsa.layers[0].core(qkv)


def test_swin_bias_values_and_padded_row_layout():
    """The drop-in's window bias equals the reference's rel-pos bias + shifted-window mask, and
    its rows are padded to a multiple of 8 keys (a 16-byte aligned row stride in fp16)."""
    torch.manual_seed(3)
    m = swin_tiny_patch4_window7(224)
    elsa_amd.patch_timm_attention(m)
    blk = m.layers[0].blocks[1]  # a shifted block: it has a mask
    attn, mask = blk.attn, blk.attn_mask
    assert mask is not None
    n, nw, h = attn.window_area, mask.shape[0], attn.num_heads
    b_win = 2 * nw
    with torch.no_grad():
        bias = attn._bias(mask, b_win, n)
        plain = attn._bias(None, b_win, n)
    dense = attn._bias(mask, b_win, n)  # the table records a gradient: dense rows
    assert dense.is_contiguous() and torch.equal(dense, bias)
    rel = attn._get_rel_pos_bias().detach()
    ref = rel + mask.view(1, nw, 1, n, n).expand(b_win // nw, -1, h, -1, -1).reshape(-1, h, n, n)
    assert bias.shape == (b_win, h, n, n) and torch.equal(bias, ref)
    assert bias.stride(-1) == 1 and bias.stride(-2) % 8 == 0 and bias.stride(-2) >= n
    assert plain.shape == (1, h, n, n) and torch.equal(plain, rel) and plain.stride(-2) % 8 == 0
    # the canonical view keeps that layout (no copy)
    from elsa_amd.attention import _canonical_bias

    meta = _canonical_bias(bias, batch=b_win, heads=h, seq_len=n, device=bias.device)
    assert meta.tensor.data_ptr() == bias.data_ptr() and meta.stride_q == bias.stride(-2)
    broadcast = rel.expand(b_win, -1, -1, -1)  # a zero batch stride is still materialised
    assert _canonical_bias(broadcast, batch=b_win, heads=h, seq_len=n, device=rel.device).stride_b == h * n * n
