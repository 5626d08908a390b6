"""The drop-in boundary on the host (no GPU): weight-layout semantics of the
atomic_ops mirror, and the prepare_triton hooks' keys, shapes and values
against the reference's hook contract (condition_gemma_inference.py:65-170,
siglip_vit_inference.py:10-101, linear_projector_inference.py:8-14)."""
import pytest
import torch

from fluxvla_amd import hooks as H
from fluxvla_amd import pi0_inference as P
from fluxvla_amd.config import tiny
from fluxvla_amd.weight_layout import (NKWeight, PatchWeight, as_nk,
                                       patch_weight_nk)
from fluxvla_amd.weights import make_state_dict

# the keys the reference's hooks return, in the reference's names
REF_VISION_KEYS = {
    'vision_patch_embedding_w', 'vision_patch_embedding_b',
    'vision_position_embedding', 'vision_attn_qkv_w', 'vision_attn_qkv_b',
    'vision_attn_o_w', 'vision_attn_o_b', 'vision_ffn_up_w', 'vision_ffn_up_b',
    'vision_ffn_down_w', 'vision_ffn_down_b', 'vision_pre_attn_norm_w',
    'vision_pre_attn_norm_b', 'vision_pre_ffn_norm_w', 'vision_pre_ffn_norm_b',
    'vision_final_norm_w', 'vision_final_norm_b'}
REF_ENCODER_KEYS = {'encoder_attn_qkv_w', 'encoder_attn_o_w',
                    'encoder_ffn_gate_w', 'encoder_ffn_up_w',
                    'encoder_ffn_down_w'}
REF_DECODER_KEYS = {
    'decoder_attn_qkv_w', 'decoder_attn_o_w', 'decoder_ffn_gate_w',
    'decoder_ffn_up_w', 'decoder_ffn_down_w', 'decoder_pre_attn_norm_mod_w',
    'decoder_pre_attn_norm_mod_b', 'decoder_pre_ffn_norm_mod_w',
    'decoder_pre_ffn_norm_mod_b', 'decoder_final_norm_mod_w',
    'decoder_final_norm_mod_b'}


def test_plain_tensor_means_in_out_and_nkweight_means_out_in():
    g = torch.Generator().manual_seed(1)
    w = torch.randn(6, 6, generator=g)             # square, not symmetric
    assert not torch.equal(w, w.t())
    assert torch.equal(as_nk(w), w.t())             # reference [in, out]
    nk = NKWeight(w)
    assert as_nk(nk) is w                           # already [out, in]
    assert nk.shape == (6, 6) and nk.size(1) == 6
    r = torch.randn(3, 5, generator=g)              # [in=3, out=5]
    assert as_nk(r).shape == (5, 3)
    t = NKWeight.from_reference(r)
    assert t.shape == r.shape and torch.equal(t.reference(), r)
    # per-layer indexing of a stacked weight keeps the tag
    st = NKWeight(torch.randn(4, 5, 3, generator=g))
    assert isinstance(st[2], NKWeight) and st[2].shape == (3, 5)
    with pytest.raises(IndexError):
        st[2][1]


def test_transposed_copy_is_cached_and_sees_in_place_updates():
    """One cache entry per weight: an in-place update is copied into the
    same [out, in] tensor (at the same address, so a graph captured over it
    reads the update after a refresh), never a second copy."""
    from fluxvla_amd import weight_layout as WL
    WL.clear_layout_cache()
    w = torch.randn(8, 4)
    a = as_nk(w)
    assert as_nk(w) is a                            # made once
    ptr = a.data_ptr()
    for scale in (2.0, 3.0):                        # two updates
        w.mul_(scale)                               # version bump
        b = as_nk(w)
        assert b is a and b.data_ptr() == ptr and torch.equal(b, w.t())
    assert len(WL._nk_cache) == 1
    # a graph replay does not call as_nk: refresh_layout_cache updates the
    # copy for it
    w.add_(1.0)
    assert WL.refresh_layout_cache() == 1 and torch.equal(a, w.t())
    assert WL.refresh_layout_cache() == 0
    WL.clear_layout_cache()


def test_patch_weight_layouts():
    cfg = tiny(vit_layers=1, llm_layers=0, exp_layers=0)
    sd = make_state_dict(cfg, seed=2)
    V = H.SigLIPViTBackboneInference.from_state_dict(sd, cfg, 'cpu').prepare_triton()
    pw = V['vision_patch_embedding_w']
    assert isinstance(pw, PatchWeight) and pw.shape == (14, 14, 3, 1152)
    conv = sd['vision_backbone.vision.vision_model.embeddings.patch_embedding.weight']
    # the reference's layout: conv [out, C, kH, kW] -> [kH, kW, C, out]
    ref = conv.permute(2, 3, 1, 0)
    assert torch.equal(pw.reference(), ref)
    kp = cfg.patch_k_pad
    assert torch.equal(patch_weight_nk(ref.contiguous(), kp), pw.nk)
    assert torch.equal(patch_weight_nk(pw, kp), pw.nk)


@pytest.mark.parametrize('pi05', [False, True])
def test_hook_keys_shapes_and_values(pi05):
    cfg = tiny(pi05=pi05, vit_layers=2, llm_layers=2, exp_layers=2)
    sd = make_state_dict(cfg, seed=3)
    V = H.SigLIPViTBackboneInference.from_state_dict(sd, cfg, 'cpu').prepare_triton()
    assert set(V) == REF_VISION_KEYS
    vh = cfg.vit_hidden
    assert V['vision_attn_qkv_w'].shape == (2, vh, 3 * vh)
    assert V['vision_ffn_up_w'].shape == (2, vh, cfg.vit_mlp)
    assert V['vision_ffn_down_w'].shape == (2, cfg.vit_mlp, vh)
    # o_proj in the reference is out_proj.weight.T: [in, out]
    o = sd['vision_backbone.vision.vision_model.encoder.layers.1.self_attn.out_proj.weight']
    assert torch.equal(V['vision_attn_o_w'][1].reference(), o.t())

    E = H.ConditionGemmaInferenceModel.from_state_dict(
        sd, cfg, 'llm_backbone', 'cpu').prepare_triton(role='llm')
    assert set(E) == REF_ENCODER_KEYS
    hq = cfg.heads * cfg.head_dim
    assert E['encoder_attn_qkv_w'].shape == (2, cfg.llm_hidden, hq + 2 * cfg.head_dim)
    assert E['encoder_attn_o_w'].shape == (2, hq, cfg.llm_hidden)
    W = P.prepare_gemma(sd, cfg, 'llm', 'cpu')
    assert torch.equal(E['encoder_attn_qkv_w'][1].nk, W['layers'][1]['qkv_w'])
    down = sd['llm_backbone.layers.0.mlp.down_proj.weight']
    assert torch.equal(E['encoder_ffn_down_w'][0].reference(), down.t())

    D = H.ConditionGemmaInferenceModel.from_state_dict(
        sd, cfg, 'llm_expert', 'cpu').prepare_triton(role='expert')
    if pi05:
        assert set(D) == REF_DECODER_KEYS
        m = sd['llm_expert.layers.1.post_attention_layernorm.dense.weight']
        assert D['decoder_pre_ffn_norm_mod_w'].shape == (2, cfg.proj_width,
                                                         3 * cfg.exp_hidden)
        assert torch.equal(D['decoder_pre_ffn_norm_mod_w'][1].reference(), m.t())
        # adaRMS layers are not folded: Q/K/V are the reference's own rows
        # (permuted), as in condition_gemma_inference.py:132-139
        q = sd['llm_expert.layers.0.self_attn.v_proj.weight']
        assert torch.equal(D['decoder_attn_qkv_w'][0].nk[-cfg.head_dim:], q)
    else:
        assert set(D) == (REF_DECODER_KEYS - {k for k in REF_DECODER_KEYS
                                              if 'norm_mod' in k}
                          | {'decoder_final_norm_scale'})
    with pytest.raises(ValueError):
        H.ConditionGemmaInferenceModel.from_state_dict(
            sd, cfg, 'llm_backbone', 'cpu').prepare_triton(role='expert')

    pj = H.LinearProjectorInference.from_state_dict(sd, 'projector', 'cpu')
    d = pj.prepare_triton(prefix='encoder_multi_modal_projector')
    assert set(d) == {'encoder_multi_modal_projector_w',
                      'encoder_multi_modal_projector_b'}
    assert torch.equal(d['encoder_multi_modal_projector_w'].reference(),
                       sd['projector.projector.weight'].t())
    # reference_layout: every NKWeight back to a plain [in, out] tensor
    R = H.reference_layout(E)
    assert all(isinstance(v, torch.Tensor) for v in R.values())
    assert torch.equal(as_nk(R['encoder_attn_o_w'][1]), E['encoder_attn_o_w'][1].nk)


def test_cache_never_serves_a_freed_weights_copy():
    """A weight freed after use and a new one allocated at the same address
    with the same shape: the new one gets its own transposed copy (the cache
    keeps its sources alive, so the address cannot be reused)."""
    from fluxvla_amd.weight_layout import clear_layout_cache
    clear_layout_cache()
    for i in range(5):
        w = torch.full((16, 8), float(i))
        w[0, 1] = 100.0 + i
        assert torch.equal(as_nk(w), w.t())
        del w
    clear_layout_cache()
