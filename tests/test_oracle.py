"""Pins of the CPU oracle (oracle/pi0_oracle.py) -- each check is chosen so a
plausible mistake (dropped term, wrong sign/index, transposed operand) fails:

* the reference's own input fixtures (tests/golden/reference_masks.npz,
  copied from test/data/models/vlas/pi0{,5}) for prefix/suffix mask
  assembly and the 2-D attention mask;
* library routines: HF transformers' GemmaDecoderLayer / GemmaRMSNorm /
  GemmaRotaryEmbedding and SiglipVisionModel (random init, same weights),
  torch scaled_dot_product_attention;
* invariants and closed forms: RoPE relative-position property, attention
  mask zeroing, adaRMS reduction, Euler loop with a constant velocity,
  brute-force mask rule on tiny inputs.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from fluxvla_amd.config import PI0Config, tiny
from fluxvla_amd.weights import make_inputs, make_state_dict
from oracle import pi0_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), 'golden',
                      'reference_masks.npz')


@pytest.fixture(scope='module')
def golden():
    return dict(np.load(GOLDEN, allow_pickle=False))


# ---------------------------------------------------------------------------
# masks and positions
# ---------------------------------------------------------------------------
def brute_force_2d(pad, att):
    """The mask rule stated in the reference (model_utils.py:77-95 after
    big_vision): i sees j iff j is not in a later block than i and both are
    valid; blocks start where att == 1.  Loops, no cumsum."""
    B, S = pad.shape
    out = torch.zeros(B, S, S, dtype=torch.bool)
    for b in range(B):
        block = []
        cur = 0
        for j in range(S):
            cur += int(att[b, j])
            block.append(cur)
        for i in range(S):
            for j in range(S):
                out[b, i, j] = (block[j] <= block[i] and bool(pad[b, i])
                                and bool(pad[b, j]))
    return out


def test_make_att_2d_masks_brute_force():
    g = torch.Generator().manual_seed(0)
    pad = torch.rand(3, 13, generator=g) > 0.2
    att = torch.rand(3, 13, generator=g) > 0.6
    assert torch.equal(O.make_att_2d_masks(pad, att), brute_force_2d(pad, att))


def test_prefix_pad_mask_from_reference_fixture(golden):
    """pi05 fixture: img_masks [1,1,0] (missing third camera) + 200-token
    prompt masks -> the stored prefix_pad_masks (968 = 3 * 256 + 200)."""
    from fluxvla_amd.pi0_inference import prefix_pad_mask
    img = torch.from_numpy(golden['pi05_img_masks'])
    lang = torch.from_numpy(golden['pi05_lang_masks'])
    want = torch.from_numpy(golden['pi05_prefix_pad_masks']).bool()
    assert torch.equal(prefix_pad_mask(img, lang, 256), want)
    # the oracle's embed_prefix builds the same mask (pi0_flowmatching.py
    # :216-247); run its mask logic on the fixture shapes
    B = img.shape[0]
    pads = [img[:, i:i + 1].expand(B, 256) for i in range(img.shape[1])]
    assert torch.equal(torch.cat(pads + [lang], 1), want)


def test_suffix_patterns_match_reference_fixtures(golden):
    from fluxvla_amd.pi0_inference import suffix_att_pattern
    pi0 = torch.from_numpy(golden['pi0_suffix_att_masks'])
    pi05 = torch.from_numpy(golden['pi05_suffix_att_masks']).bool()
    cfg0 = PI0Config()
    cfg5 = PI0Config(pi05=True, n_action_steps=pi05.shape[1])
    assert pi0.shape[1] == cfg0.suffix_len
    for row in pi0:
        assert row.int().tolist() == suffix_att_pattern(cfg0)
    for row in pi05:
        assert row.int().tolist() == suffix_att_pattern(cfg5)
    # and the oracle's embed_suffix emits the same patterns
    cfg = tiny()
    sd = make_state_dict(cfg.scaled(vit_layers=0, llm_layers=0, exp_layers=0))
    x = torch.zeros(2, cfg.n_action_steps, cfg.max_action_dim)
    _, _, att, _ = O.embed_suffix(sd, cfg, torch.zeros(2, 32), x,
                                  torch.tensor([0.5, 0.5]))
    assert torch.equal(att, pi0)


@pytest.mark.parametrize('which', ['pi0', 'pi05'])
def test_kernel_mask_encoding_equals_2d_mask(golden, which):
    """Product encoding kgrp[j] <= qgrp[i] == the oracle's full 2-D mask of
    denoise_step (prefix pad 2-D | suffix block mask) on the reference's
    own masks, and the prefix mask for valid query rows; positions equal
    cumsum-based position ids."""
    from fluxvla_amd.pi0_inference import attention_groups
    ppad = torch.from_numpy(golden[f'{which}_prefix_pad_masks']).bool()
    patt = torch.from_numpy(golden[f'{which}_prefix_att_masks']).bool()
    spad = torch.from_numpy(golden[f'{which}_suffix_pad_masks']).bool()
    satt = torch.from_numpy(golden[f'{which}_suffix_att_masks']).bool()
    assert not patt.any()
    B, S = ppad.shape
    Ss = spad.shape[1]
    kgrp, qg_pre, qg_suf, pos_pre, pos_suf = attention_groups(
        ppad, satt[0].int().tolist())
    # suffix rows (denoise_step, pi0_flowmatching.py:796-813)
    full = torch.cat([ppad[:, None, :].expand(B, Ss, S),
                      O.make_att_2d_masks(spad, satt)], dim=2)
    enc = kgrp[:, None, :] <= qg_suf[:, :, None]
    assert torch.equal(enc, full)
    # prefix rows, valid queries (predict_action :728-730)
    pm = O.make_att_2d_masks(ppad, patt)
    enc_p = kgrp[:, None, :S] <= qg_pre[:, :, None]
    assert torch.equal(enc_p & ppad[:, :, None], pm)
    assert torch.equal(pos_pre.long(), torch.cumsum(ppad.long(), 1) - 1)
    want_suf = ppad.sum(-1, keepdim=True) + torch.cumsum(spad.long(), 1) - 1
    assert torch.equal(pos_suf.long(), want_suf)


# ---------------------------------------------------------------------------
# Gemma: against HF transformers' Gemma modules (library routine)
# ---------------------------------------------------------------------------
def _small_gemma_cfg():
    return tiny(llm_hidden=64, llm_mlp=96, heads=4, head_dim=16,
                llm_layers=2)


def _hf_gemma(cfg):
    from transformers import GemmaConfig
    from transformers.models.gemma.modeling_gemma import (
        GemmaDecoderLayer, GemmaRMSNorm, GemmaRotaryEmbedding)
    hc = GemmaConfig(hidden_size=cfg.llm_hidden,
                     intermediate_size=cfg.llm_mlp,
                     num_attention_heads=cfg.heads, num_key_value_heads=1,
                     head_dim=cfg.head_dim, num_hidden_layers=cfg.llm_layers,
                     vocab_size=16, rms_norm_eps=cfg.rms_eps,
                     rope_theta=cfg.rope_theta,
                     hidden_act='gelu_pytorch_tanh',
                     hidden_activation='gelu_pytorch_tanh',
                     attention_dropout=0.0)
    hc._attn_implementation = 'eager'
    layers = [GemmaDecoderLayer(hc, i) for i in range(cfg.llm_layers)]
    return hc, layers, GemmaRMSNorm(cfg.llm_hidden, eps=cfg.rms_eps), \
        GemmaRotaryEmbedding(hc)


def test_gemma_layers_match_hf():
    cfg = _small_gemma_cfg()
    sd = {k: v.float() for k, v in make_state_dict(cfg, seed=3).items()
          if k.startswith('llm_backbone.')}
    hc, layers, norm, rot = _hf_gemma(cfg)
    for i, layer in enumerate(layers):
        pre = f'llm_backbone.layers.{i}.'
        layer.load_state_dict({k[len(pre):]: v for k, v in sd.items()
                               if k.startswith(pre)})
    norm.load_state_dict({'weight': sd['llm_backbone.norm.weight']})
    g = torch.Generator().manual_seed(1)
    B, S = 2, 11
    x = torch.randn(B, S, cfg.llm_hidden, generator=g)
    pad = torch.ones(B, S, dtype=torch.bool)
    pad[1, 8:] = False
    att = torch.zeros(B, S, dtype=torch.bool)
    att[:, 5] = True  # two blocks: bidirectional inside, causal across
    mask = O.make_att_2d_masks(pad, att)
    pos = torch.cumsum(pad.long(), 1) - 1
    got, kvs = O.gemma_model(sd, 'llm_backbone', cfg.llm_layers, x, pos, mask,
                             cfg)
    add = torch.zeros(B, 1, S, S).masked_fill(~mask[:, None], O.BF16_MIN)
    h = x
    with torch.no_grad():
        pe = rot(h, pos)
        for layer in layers:
            out = layer(h, attention_mask=add, position_ids=pos,
                        position_embeddings=pe)
            h = out[0] if isinstance(out, tuple) else out
        ref = norm(h)
    valid = pad[:, :, None].expand_as(ref)
    err = (got - ref)[valid].abs().max().item()
    assert err <= 1e-4 * ref.abs().max().item()
    # the KV of layer 0 is the rotated K / plain V of the normed input
    assert kvs[0][0].shape == (B, 1, S, cfg.head_dim)


def test_rope_relative_position_and_norm():
    """<R(p) q, R(p') k> depends only on p - p'; rotations keep norms."""
    D = 32
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, 1, 1, D, generator=g)
    k = torch.randn(1, 1, 1, D, generator=g)

    def dot(p, pk):
        cq, sq = O.rope_cos_sin(torch.tensor([[p]]), D, 10000.0)
        ck, sk = O.rope_cos_sin(torch.tensor([[pk]]), D, 10000.0)
        rq, _ = O.apply_rope(q, q, cq, sq)
        rk, _ = O.apply_rope(k, k, ck, sk)
        return (rq * rk).sum().item(), rq.norm().item()

    a, na = dot(7, 3)
    b, nb = dot(107, 103)
    assert abs(a - b) < 1e-3
    assert abs(na - q.norm().item()) < 1e-4


def test_interleaved_rope_layout_preserves_scores():
    """Permuting Q/K rows to pair-interleaved order (the kernels' layout,
    condition_gemma_inference.py:46-63) leaves Q K^T unchanged."""
    from fluxvla_amd.pi0_inference import interleave_rows
    D = 16
    perm = interleave_rows(D)
    assert sorted(perm.tolist()) == list(range(D))
    # pair (i, i + D/2) lands on (2i, 2i + 1)
    for i in range(D // 2):
        assert perm[2 * i].item() == i and perm[2 * i + 1].item() == i + D // 2
    g = torch.Generator().manual_seed(3)
    q = torch.randn(5, D, generator=g)
    k = torch.randn(7, D, generator=g)
    assert torch.allclose(q @ k.t(), q[:, perm] @ k[:, perm].t(), atol=1e-6)


def test_attention_matches_sdpa_and_masks_zero():
    g = torch.Generator().manual_seed(4)
    B, H, Sq, Sk, D = 2, 4, 5, 9, 16
    q = torch.randn(B, H, Sq, D, generator=g)
    k = torch.randn(B, 1, Sk, D, generator=g)
    v = torch.randn(B, 1, Sk, D, generator=g)
    mask = torch.rand(B, Sq, Sk, generator=g) > 0.3
    mask[:, :, 0] = True
    got = O.attention(q, k, v, mask, D**-0.5)
    ref = F.scaled_dot_product_attention(
        q, k.expand(-1, H, -1, -1), v.expand(-1, H, -1, -1),
        attn_mask=mask[:, None])
    assert torch.allclose(got, ref, atol=1e-5)
    # perturbing masked values changes nothing
    v2 = v.clone()
    v2[~mask.any(1)[:, None, :, None].expand_as(v2)] += 100.0
    assert torch.allclose(O.attention(q, k, v2, mask, D**-0.5), got,
                          atol=1e-5)


def test_adarms_reduces_to_plain_rms():
    """Zero modulation -> plain RMSNorm with w = 0 (condition_gemma.py:70)."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 4, 16, generator=g)
    cond = torch.randn(3, 8, generator=g)
    y, gate = O.ada_rms_norm(x, cond, torch.zeros(48, 8), torch.zeros(48),
                             1e-6)
    assert torch.allclose(y, O.gemma_rms_norm(x, torch.zeros(16), 1e-6))
    assert gate.abs().max().item() == 0.0
    # and RMSNorm output has unit RMS when w = 0
    r = O.gemma_rms_norm(x, torch.zeros(16), 0.0)
    assert torch.allclose(r.pow(2).mean(-1), torch.ones(3, 4), atol=1e-5)


# ---------------------------------------------------------------------------
# SigLIP: against HF transformers' SiglipVisionModel
# ---------------------------------------------------------------------------
def test_siglip_tower_matches_hf():
    from transformers import SiglipVisionConfig, SiglipVisionModel
    cfg = tiny(vit_hidden=64, vit_heads=4, vit_layers=2, vit_mlp=96,
               image_size=28, patch=14)
    sd = make_state_dict(cfg.scaled(llm_layers=0, exp_layers=0), seed=6)
    sd = {k: v.float() for k, v in sd.items()}
    hc = SiglipVisionConfig(hidden_size=64, intermediate_size=96,
                            num_attention_heads=4, num_hidden_layers=2,
                            image_size=28, patch_size=14, layer_norm_eps=1e-6,
                            hidden_act='gelu_pytorch_tanh',
                            attention_dropout=0.0)
    hc._attn_implementation = 'eager'
    model = SiglipVisionModel(hc).eval()
    # transformers 4.53.2 (the reference's pin) nests the tower under
    # `vision_model.`; 5.x does not -- accept whichever this install uses.
    nested = any(k.startswith('vision_model.') for k in model.state_dict())
    pre = 'vision_backbone.vision.' + ('' if nested else 'vision_model.')
    hf_sd = {k[len(pre):]: v for k, v in sd.items() if k.startswith(pre)}
    missing, unexpected = model.load_state_dict(hf_sd, strict=False)
    assert not unexpected
    assert all('head' in m or 'position_ids' in m for m in missing), missing
    g = torch.Generator().manual_seed(7)
    px = torch.rand(2, 3, 28, 28, generator=g) * 2 - 1
    with torch.no_grad():
        ref = model(pixel_values=px).last_hidden_state
    got = O.siglip_tower(sd, px, cfg)
    assert (got - ref).abs().max().item() <= 1e-4 * ref.abs().max().item()


# ---------------------------------------------------------------------------
# time embedding and the Euler loop
# ---------------------------------------------------------------------------
def test_sinusoidal_embedding_closed_form():
    d = 16
    e0 = O.sinusoidal_pos_embedding(torch.tensor([0.0]), d, 4e-3, 4.0)
    assert torch.allclose(e0[0, :8], torch.zeros(8))
    assert torch.allclose(e0[0, 8:], torch.ones(8))
    # the slowest component has period max_period: sin(2 pi t / 4)
    t = torch.tensor([0.5])
    e = O.sinusoidal_pos_embedding(t, d, 4e-3, 4.0)
    assert abs(e[0, 7].item() - math.sin(2 * math.pi * 0.5 / 4.0)) < 1e-6
    assert abs(e[0, 0].item() - math.sin(2 * math.pi * 0.5 / 4e-3)) < 1e-3


@pytest.mark.parametrize('n', [1, 2, 3, 7, 10, 16, 25])
def test_euler_schedule(n):
    """Exactly n steps, starting at t = 1, ending near 1/n, decreasing."""
    from fluxvla_amd.pi0_inference import euler_times
    ts = O.euler_times(n)
    assert len(ts) == n and ts[0] == 1.0
    assert abs(ts[-1] - 1.0 / n) < 1e-5
    assert all(a > b for a, b in zip(ts, ts[1:]))
    assert euler_times(n)[0] == ts


def test_predict_action_constant_velocity():
    """Zero expert weights and zero action_out weight make v = bias for
    every step: the loop then returns noise - bias (sum of dt = -1)."""
    cfg = tiny(vit_layers=1, llm_layers=1, exp_layers=1)
    sd = make_state_dict(cfg, seed=8)
    for k in list(sd):
        if k.startswith('llm_expert.') or k == 'action_out_proj.projector.weight':
            sd[k] = torch.zeros_like(sd[k])
    inp = make_inputs(cfg, batch=1, seed=9)
    out = O.predict_action(sd, cfg, inp['images'], inp['lang_tokens'],
                           inp['states'], noise=inp['noise'], num_steps=4)
    bias = sd['action_out_proj.projector.bias'].float()
    assert torch.allclose(out, inp['noise'] - bias, atol=1e-5)


def test_one_step_equals_single_denoise():
    cfg = tiny(vit_layers=1, llm_layers=1, exp_layers=1)
    sd = make_state_dict(cfg, seed=10)
    inp = make_inputs(cfg, batch=1, seed=11)
    out = O.predict_action(sd, cfg, inp['images'], inp['lang_tokens'],
                           inp['states'], noise=inp['noise'], num_steps=1)
    kvs, pad = O.prefix_forward(sd, cfg, inp['images'], inp['lang_tokens'],
                                torch.ones(1, 3, dtype=torch.bool),
                                torch.ones(1, 48, dtype=torch.bool))
    v = O.denoise_step(sd, cfg, inp['states'], pad, kvs, inp['noise'],
                       torch.tensor([1.0]))
    assert torch.allclose(out, inp['noise'] - v, atol=1e-5)


# ---------------------------------------------------------------------------
# closed forms that pin the modulation order, the gated residual, the suffix
# embeddings and the prefix language scale (each with a planted mistake that
# the same check must reject)
# ---------------------------------------------------------------------------
def _unit_rows(n, d):
    """Rows of +-1 entries: mean(x^2) = 1 exactly, so rms-normalised x is
    x / sqrt(1 + eps)."""
    g = torch.Generator().manual_seed(40)
    return torch.where(torch.rand(n, d, generator=g) > 0.5, 1.0, -1.0)


def _adarms_closed_form_ok(fn):
    """dense weight 0, bias [scale = 0.5 | shift = 2 | gate = -3]: for x =
    +-1 the output must be n * 1.5 + 2 with n = x / sqrt(1 + eps), i.e.
    ~3.5 for +1 and ~0.5 for -1 (condition_gemma.py:136-145 chunks the
    modulation as scale, shift, gate), and the gate -3 everywhere."""
    eps = 1e-6
    d = 8
    x = _unit_rows(6, d)[None]
    cond = torch.randn(1, 5, generator=torch.Generator().manual_seed(41))
    b = torch.cat([torch.full((d,), 0.5), torch.full((d,), 2.0),
                   torch.full((d,), -3.0)])
    y, gate = fn(x, cond, torch.zeros(3 * d, 5), b, eps)
    n = 1.0 / math.sqrt(1.0 + eps)
    want = torch.where(x > 0, 1.5 * n + 2.0, -1.5 * n + 2.0)
    return (torch.allclose(y, want, atol=1e-6) and
            torch.allclose(gate, torch.full_like(gate, -3.0)))


def test_adarms_modulation_order_closed_form():
    assert _adarms_closed_form_ok(O.ada_rms_norm)

    # planted mistakes: scale/shift swapped, gate taken from the wrong chunk
    def swapped(x, cond, w, b, eps):
        d = b.numel() // 3
        b2 = torch.cat([b[d:2 * d], b[:d], b[2 * d:]])
        return O.ada_rms_norm(x, cond, w, b2, eps)

    def gate_first(x, cond, w, b, eps):
        d = b.numel() // 3
        b2 = torch.cat([b[2 * d:], b[d:2 * d], b[:d]])
        return O.ada_rms_norm(x, cond, w, b2, eps)

    assert not _adarms_closed_form_ok(swapped)
    assert not _adarms_closed_form_ok(gate_first)


def _pi05_layer_sd(cfg, gate_value):
    """One adaRMS expert layer whose dense modulations are zero except the
    gate bias (scale = shift = 0, gate = gate_value)."""
    sd = {k: v.float() for k, v in make_state_dict(cfg, seed=42).items()
          if k.startswith('llm_expert.layers.0.')}
    hid = cfg.exp_hidden
    for norm in ('input_layernorm', 'post_attention_layernorm'):
        pre = f'llm_expert.layers.0.{norm}.dense'
        sd[pre + '.weight'] = torch.zeros_like(sd[pre + '.weight'])
        sd[pre + '.bias'] = torch.cat([torch.zeros(2 * hid),
                                       torch.full((hid,), gate_value)])
    return sd


def test_gated_residual_closed_form():
    """condition_gemma.py:319-337 (`x + y * gate`): gate 0 leaves the stream
    unchanged; gate 1 with scale = shift = 0 equals the ungated layer with a
    plain RMSNorm of weight 0 (1 + w = 1)."""
    cfg = tiny(pi05=True, exp_hidden=32, exp_mlp=48, heads=2, head_dim=8,
               proj_width=16, exp_layers=1)
    g = torch.Generator().manual_seed(43)
    B, S = 1, 5
    h = torch.randn(B, S, cfg.exp_hidden, generator=g)
    cond = torch.randn(B, cfg.proj_width, generator=g)
    pos = torch.arange(S)[None]
    cos, sin = O.rope_cos_sin(pos, cfg.head_dim, cfg.rope_theta)
    pre = 'llm_expert.layers.0'
    out0, _ = O.gemma_layer(_pi05_layer_sd(cfg, 0.0), pre, h, cos, sin, None,
                            None, cond, cfg)
    assert torch.equal(out0, h)
    sd1 = _pi05_layer_sd(cfg, 1.0)
    out1, _ = O.gemma_layer(sd1, pre, h, cos, sin, None, None, cond, cfg)
    plain = dict(sd1)
    for norm in ('input_layernorm', 'post_attention_layernorm'):
        plain[f'{pre}.{norm}.weight'] = torch.zeros(cfg.exp_hidden)
    ref, _ = O.gemma_layer(plain, pre, h, cos, sin, None, None, None, cfg)
    assert torch.allclose(out1, ref, atol=1e-5)
    assert not torch.allclose(out1, h, atol=1e-3)
    # gate 2: the attention and MLP deltas of the first half double
    out2, _ = O.gemma_layer(_pi05_layer_sd(cfg, 2.0), pre, h, cos, sin, None,
                            None, cond, cfg)
    assert not torch.allclose(out2, out1, atol=1e-3)


def _suffix_cfg(pi05):
    return tiny(pi05=pi05, proj_width=32, exp_hidden=32, vit_layers=0,
                llm_layers=0, exp_layers=0)


def _eye_sd(cfg):
    """Projection weights that expose the suffix embedding's structure:
    action_in / state_proj copy their 32 inputs into the first 32 outputs,
    action_time_mlp_in is [I | 0] (action half only), mlp_out is 2 I, time
    MLPs are the identity; every bias is zero."""
    w, ad = cfg.proj_width, cfg.max_action_dim
    sd = {}
    eye_in = torch.zeros(w, ad)
    eye_in[:ad, :ad] = torch.eye(ad)
    for nm in ('action_in_proj', 'state_proj'):
        sd[f'{nm}.projector.weight'] = eye_in.clone()
        sd[f'{nm}.projector.bias'] = torch.zeros(w)
    sd['action_time_mlp_in.projector.weight'] = torch.cat(
        [torch.eye(w), torch.zeros(w, w)], 1)
    sd['action_time_mlp_in.projector.bias'] = torch.zeros(w)
    sd['action_time_mlp_out.projector.weight'] = 2 * torch.eye(w)
    sd['action_time_mlp_out.projector.bias'] = torch.zeros(w)
    for nm in ('time_mlp_in', 'time_mlp_out'):
        sd[f'{nm}.projector.weight'] = torch.eye(w)
        sd[f'{nm}.projector.bias'] = torch.zeros(w)
    return sd


def test_pi0_embed_suffix_closed_form():
    """pi0_flowmatching.py:252-321: row 0 is state_proj(state); rows 1.. are
    mlp_out(silu(mlp_in(cat([action_in(x_t), temb])))), so with the weights
    of _eye_sd the action rows are 2 * silu(x_t) on the first 32 dims and 0
    elsewhere; with mlp_in = [0 | I] they become 2 * silu(temb)."""
    cfg = _suffix_cfg(False)
    sd = _eye_sd(cfg)
    g = torch.Generator().manual_seed(44)
    B, n = 2, cfg.n_action_steps
    x_t = torch.randn(B, n, cfg.max_action_dim, generator=g)
    states = torch.rand(B, cfg.state_dim, generator=g) * 2 - 1
    t = torch.tensor([0.7, 0.3])
    embs, pad, att, cond = O.embed_suffix(sd, cfg, states, x_t, t)
    assert cond is None and embs.shape == (B, n + 1, cfg.proj_width)
    assert torch.equal(embs[:, 0], states)            # state row first
    silu = x_t * torch.sigmoid(x_t)
    assert torch.allclose(embs[:, 1:], 2 * silu, atol=1e-6)
    # planted mistakes that the same closed form must reject
    assert not torch.allclose(embs[:, 1:], torch.nn.functional.silu(2 * x_t),
                              atol=1e-3)              # SiLU after mlp_out
    # time half: mlp_in = [0 | I]
    sd['action_time_mlp_in.projector.weight'] = torch.cat(
        [torch.zeros(cfg.proj_width, cfg.proj_width),
         torch.eye(cfg.proj_width)], 1)
    embs, _, _, _ = O.embed_suffix(sd, cfg, states, x_t, t)
    temb = O.sinusoidal_pos_embedding(t, cfg.proj_width, 4e-3, 4.0)
    want = 2 * temb * torch.sigmoid(temb)
    assert torch.allclose(embs[:, 1:], want[:, None].expand(B, n, -1),
                          atol=1e-6)


def test_pi05_embed_suffix_closed_form():
    """pi05_flowmatching.py:68-127: the tokens are action_in(x_t) alone and
    the adaRMS condition is silu(mlp_out(silu(mlp_in(temb)))); with identity
    time MLPs it is silu(silu(temb)), and with mlp_in = 2 I it is
    silu(silu(2 temb)) (not 2 silu(...): the scale sits inside)."""
    cfg = _suffix_cfg(True)
    sd = _eye_sd(cfg)
    g = torch.Generator().manual_seed(45)
    B, n = 2, cfg.n_action_steps
    x_t = torch.randn(B, n, cfg.max_action_dim, generator=g)
    t = torch.tensor([1.0, 0.4])
    embs, pad, att, cond = O.embed_suffix(sd, cfg, torch.zeros(B, 32), x_t, t)
    assert embs.shape == (B, n, cfg.proj_width)
    assert torch.equal(embs[..., :cfg.max_action_dim], x_t)
    assert torch.equal(embs[..., cfg.max_action_dim:],
                       torch.zeros(B, n, cfg.proj_width - cfg.max_action_dim))
    temb = O.sinusoidal_pos_embedding(t, cfg.proj_width, 4e-3, 4.0)

    def silu(v):
        return v * torch.sigmoid(v)
    assert torch.allclose(cond, silu(silu(temb)), atol=1e-6)
    sd['time_mlp_in.projector.weight'] = 2 * torch.eye(cfg.proj_width)
    _, _, _, cond2 = O.embed_suffix(sd, cfg, torch.zeros(B, 32), x_t, t)
    assert torch.allclose(cond2, silu(silu(2 * temb)), atol=1e-6)
    assert not torch.allclose(cond2, 2 * silu(silu(temb)), atol=1e-3)


def test_embed_prefix_language_scale_and_image_rows():
    """pi0_flowmatching.py:204-250: language rows are embed_tokens[ids] *
    sqrt(width) (table row i filled with i / 64 -> ids / 64 * sqrt(width));
    image rows carry no such scale (projector weight 0, bias c -> exactly
    c)."""
    cfg = tiny(vit_hidden=64, vit_heads=4, vit_layers=1, vit_mlp=96,
               llm_hidden=64, image_size=28, patch=14, vocab=50,
               max_prompt_len=6, llm_layers=0, exp_layers=0)
    sd = {k: v.float() for k, v in make_state_dict(cfg, seed=46).items()}
    sd['llm_backbone.embed_tokens.weight'] = (
        torch.arange(cfg.vocab, dtype=torch.float32)[:, None] / 64.0
    ).expand(cfg.vocab, cfg.llm_hidden).contiguous()
    c = torch.linspace(-1, 1, cfg.llm_hidden)
    sd['projector.projector.weight'] = torch.zeros(cfg.llm_hidden,
                                                   cfg.vit_hidden)
    sd['projector.projector.bias'] = c
    g = torch.Generator().manual_seed(47)
    B = 2
    images = torch.rand(B, 3 * cfg.n_views, 28, 28, generator=g) * 2 - 1
    ids = torch.randint(0, cfg.vocab, (B, cfg.max_prompt_len), generator=g)
    img_masks = torch.ones(B, cfg.n_views, dtype=torch.bool)
    lang_masks = torch.ones(B, cfg.max_prompt_len, dtype=torch.bool)
    embs, pad, att = O.embed_prefix(sd, cfg, images, ids, img_masks,
                                    lang_masks)
    n_img = cfg.n_views * cfg.num_patches
    assert embs.shape == (B, n_img + cfg.max_prompt_len, cfg.llm_hidden)
    assert torch.equal(embs[:, :n_img], c.expand(B, n_img, -1))
    want = (ids.float() / 64.0 * 8.0)[..., None].expand(-1, -1, cfg.llm_hidden)
    assert torch.allclose(embs[:, n_img:], want, atol=1e-6)   # sqrt(64) = 8
    assert not att.any() and pad.all()


# ---------------------------------------------------------------------------
# Real-time chunking (pi0_flowmatching.py:651-700, rtc_guidance.py:28-155)
# ---------------------------------------------------------------------------
def test_prefix_weights_closed_form():
    """Locked prefix 1; the decay runs from 1 at prefix_len to its end value
    at decay_end - 1 (exp: exp(-3), linear: 0); zero after decay_end."""
    w = O.compute_prefix_weights(50, 5, 15, 'exp')
    assert torch.equal(w[:5], torch.ones(5))
    assert w[5].item() == 1.0
    assert abs(w[14].item() - math.exp(-3.0)) < 1e-7
    assert abs(w[10].item() - math.exp(-3.0 * 5 / 9)) < 1e-7
    assert torch.equal(w[15:], torch.zeros(35))
    assert torch.all(w[5:15][1:] < w[5:15][:-1])  # strictly decaying
    lin = O.compute_prefix_weights(50, 5, 15, 'linear')
    assert abs(lin[14].item()) < 1e-7 and abs(lin[8].item() - 2 / 3) < 1e-7
    assert torch.equal(O.compute_prefix_weights(50, 5, 15, 'ones')[:15],
                       torch.ones(15))
    z = O.compute_prefix_weights(50, 5, 15, 'zeros')
    assert torch.equal(z, torch.cat([torch.ones(5), torch.zeros(45)]))
    # no prefix: all zero; decay clipped at the chunk end; prefix clipped
    assert torch.equal(O.compute_prefix_weights(50, 0, 10), torch.zeros(50))
    assert O.compute_prefix_weights(10, 8, 20)[9].item() > 0
    assert torch.equal(O.compute_prefix_weights(10, 12, 24), torch.ones(10))
    # a one-long decay is weight 1 (f = 0)
    assert O.compute_prefix_weights(50, 5, 6, 'exp')[5].item() == 1.0
    with pytest.raises(ValueError):
        O.compute_prefix_weights(50, 5, 15, 'cosine')


def test_guidance_weight_closed_form():
    """(1-t)/t * (t^2 + (1-t)^2)/(1-t)^2: 2 at t = 1/2, 82/9 at t = 0.9,
    capped by the maximum, and the maximum at t = 0 (pure noise)."""
    assert abs(O.compute_guidance_weight(0.5, 100.0) - 2.0) < 1e-12
    assert abs(O.compute_guidance_weight(0.9, 100.0) - 82.0 / 9.0) < 1e-9
    assert O.compute_guidance_weight(0.9, 5.0) == 5.0
    assert O.compute_guidance_weight(0.0, 5.0) == 5.0
    assert abs(O.compute_guidance_weight(0.25, 100.0) -
               3.0 * (0.0625 + 0.5625) / 0.5625) < 1e-12


def _elementwise_denoiser(calls):
    """v = -(x + t): rows are independent, time enters per position."""
    def denoise(x, t):
        calls.append((x.clone(), t.clone()))
        tt = t[:, :, None] if t.dim() == 2 else t[:, None, None]
        return -(x + tt)
    return denoise


def test_prefix_rtc_loop_contract():
    """Every denoise call sees the previous chunk on the locked rows and time
    0 there (the current time elsewhere); the result holds the previous
    chunk on the locked rows and, on the others, what the plain loop gives
    for a row-independent denoiser fed the same per-position times."""
    g = torch.Generator().manual_seed(0)
    B, T, D, p = 2, 50, 32, 7
    noise = torch.randn(B, T, D, generator=g)
    prev = torch.randn(B, 30, D, generator=g)
    dt = torch.tensor(-0.1)
    calls = []
    out = O.euler_prefix_rtc(noise.clone(), _elementwise_denoiser(calls), B,
                             dt, prev, p, T)
    times = O.euler_times(10)
    assert len(calls) == 10
    for (x, t), time in zip(calls, times):
        assert torch.equal(x[:, :p], prev[:, :p])
        assert torch.equal(t[:, :p], torch.zeros(B, p))
        assert torch.all(t[:, p:] == time)
    assert torch.equal(out[:, :p], prev[:, :p])
    # unlocked rows: x <- x + dt * -(x + time), a scalar recursion per value
    x = noise[:, p:].clone()
    for time in times:
        x = x + dt * -(x + time)
    assert torch.allclose(out[:, p:], x, atol=1e-6)


def test_guidance_rtc_constant_velocity():
    """Constant velocity c: the plain loop ends at noise - c, which is also
    the clean-chunk estimate x_1 = x - time * c at every step.  Guided
    towards exactly that chunk the correction vanishes; guided towards it
    plus delta on a row of weight w, the distance to the target shrinks by
    (1 + dt * gw_k * w) per step, a row of weight 0 keeps the plain result,
    and rows past the previous chunk are not guided."""
    g = torch.Generator().manual_seed(1)
    B, T, D = 1, 50, 32
    noise = torch.randn(B, T, D, generator=g)
    c = torch.randn(B, T, D, generator=g)
    dt = torch.tensor(-0.1)

    def denoise(x, t):
        return c.clone()

    plain = noise - c
    rc = {'method': 'guidance', 'max_guidance_weight': 5.0, 'decay_end': 12,
          'schedule': 'linear'}
    out = O.euler_guidance_rtc(noise.clone(), denoise, B, dt, plain.clone(), 4,
                               rc, T)
    assert torch.allclose(out, plain, atol=1e-5)
    delta = torch.randn(B, 40, D, generator=g)
    prev = plain[:, :40] + delta
    out = O.euler_guidance_rtc(noise.clone(), denoise, B, dt, prev, 4, rc, T)
    w = O.compute_prefix_weights(T, 4, 12, 'linear')
    times = O.euler_times(10)
    gws = [O.compute_guidance_weight(1.0 - tm, 5.0) for tm in times]
    assert gws[0] == 5.0
    for r in (0, 3, 6, 10, 20, 45):
        f = 1.0
        for gw in gws:
            f *= 1.0 - 0.1 * gw * (w[r].item() if r < 40 else 0.0)
        d = delta[:, r] if r < 40 else torch.zeros(B, D)
        expect = plain[:, r] + d * (1.0 - f)
        assert torch.allclose(out[:, r], expect, atol=1e-4), r
    # gw is the maximum at both ends of the schedule and 2 at time 1/2
    assert gws[-1] == 5.0 and abs(gws[5] - 2.0) < 1e-5
    # a weight-1 row closes 1 - 0.5^2 * (1 - 0.1 * 4.25)^2 * ... of delta;
    # with the sign of the correction flipped it would grow instead
    assert (out[:, 0] - prev[:, 0]).abs().max() < 0.05 * delta[:, 0].abs().max()


def test_guidance_without_previous_rows():
    """A previous chunk with no rows guides nothing (rtc_guidance.py:142-144)."""
    x = torch.randn(1, 50, 32)
    v = torch.randn(1, 50, 32)
    got = O.apply_rtc_guidance(x, lambda z: v.clone(), torch.zeros(1, 0, 32),
                               torch.ones(50), 0.3, 5.0)
    assert torch.equal(got, v)


def test_rtc_method_selection():
    """predict_action runs RTC only with prev_actions, prefix_len > 0 and a
    config; shorter action dims are zero-padded with ori_action_dim."""
    cfg = PI0Config(ori_action_dim=14)
    prev = torch.ones(1, 5, 14)
    p, m = O.rtc_inputs(cfg, prev, 3, {'method': 'guidance'})
    assert m == 'guidance' and p.shape == (1, 5, 32)
    assert torch.equal(p[..., 14:], torch.zeros(1, 5, 18))
    assert O.rtc_inputs(cfg, prev, 3, {})[1] is None
    assert O.rtc_inputs(cfg, prev, 0, {'method': 'prefix'})[1] is None
    assert O.rtc_inputs(cfg, None, 3, {'method': 'prefix'})[1] is None
    assert O.rtc_inputs(cfg, prev, 3, {'enabled': True})[1] == 'prefix'
    assert O.rtc_inputs(PI0Config(), prev, 3, {})[0].shape[-1] == 14


# ---------------------------------------------------------------------------
# denoise_step: suffix positions and the output rows
# ---------------------------------------------------------------------------
def _joint_cfg():
    """PI0 with the expert shaped like the prefix LLM, so one Gemma stack
    can run the joint [prefix | suffix] sequence."""
    return tiny(llm_hidden=64, exp_hidden=64, llm_mlp=96, exp_mlp=96,
                heads=4, head_dim=16, proj_width=64, llm_layers=2,
                exp_layers=2, vit_layers=0)


def _joint_setup():
    cfg = _joint_cfg()
    sd = {k: v.float() for k, v in make_state_dict(cfg, seed=50).items()}
    # sharp attention (scores of order 10), so relative positions matter
    for k in list(sd):
        if '.q_proj.' in k or '.k_proj.' in k:
            sd[k] = sd[k] * 25
    # the expert becomes a copy of the prefix LLM (layers and final norm)
    for k in list(sd):
        if k.startswith('llm_backbone.layers.') or k == 'llm_backbone.norm.weight':
            sd['llm_expert.' + k[len('llm_backbone.'):]] = sd[k].clone()
    g = torch.Generator().manual_seed(51)
    B, Sp = 2, 13
    prefix = torch.randn(B, Sp, cfg.llm_hidden, generator=g)
    ppad = torch.ones(B, Sp, dtype=torch.bool)
    ppad[0, 4:7] = False        # a masked camera in the middle
    ppad[1, 10:] = False        # a padded prompt tail
    patt = torch.zeros(B, Sp, dtype=torch.bool)
    states = torch.rand(B, cfg.state_dim, generator=g) * 2 - 1
    x_t = torch.randn(B, cfg.n_action_steps, cfg.max_action_dim, generator=g)
    t = torch.tensor([0.8, 0.3])
    return cfg, sd, prefix, ppad, patt, states, x_t, t


def _joint_reference(cfg, sd, prefix, ppad, patt, states, x_t, t):
    """The training forward's joint pass (pi0_flowmatching.py:590-628): one
    sequence [prefix | suffix], positions cumsum(joint pad) - 1 and the
    joint make_att_2d_masks; with the expert equal to the LLM the per-tower
    layers (:323-434) are one Gemma stack.  The velocity is
    action_out_proj(suffix_out[:, -n_action_steps:])."""
    s_emb, spad, satt, _ = O.embed_suffix(sd, cfg, states, x_t, t)
    embs = torch.cat([prefix, s_emb], 1)
    pad = torch.cat([ppad, spad], 1)
    att = torch.cat([patt, satt], 1)
    pos = torch.cumsum(pad.long(), 1) - 1
    h, _ = O.gemma_model(sd, 'llm_backbone', cfg.llm_layers, embs, pos,
                         O.make_att_2d_masks(pad, att), cfg)
    out = h[:, -cfg.n_action_steps:]
    return O.linear(out, sd['action_out_proj.projector.weight'],
                    sd['action_out_proj.projector.bias'])


def _cached_velocity(denoise, cfg, sd, prefix, ppad, patt, states, x_t, t):
    """predict_action's cache (pi0_flowmatching.py:722-742) then one
    denoise step."""
    pos = torch.cumsum(ppad.long(), 1) - 1
    _, kvs = O.gemma_model(sd, 'llm_backbone', cfg.llm_layers, prefix, pos,
                           O.make_att_2d_masks(ppad, patt), cfg,
                           kv_only_last=True)
    return denoise(sd, cfg, states, ppad, kvs, x_t, t)


def _planted_denoise(pos_shift=0, first_rows=False):
    """denoise_step with one planted mistake: suffix positions shifted by
    pos_shift, or the first n_action_steps rows taken instead of the last."""
    def fn(P, cfg, states, prefix_pad, kvs, x_t, timestep):
        embs, spad, satt, cond = O.embed_suffix(P, cfg, states, x_t, timestep)
        B, Ss = spad.shape
        full = torch.cat([prefix_pad[:, None, :].expand(B, Ss, -1),
                          O.make_att_2d_masks(spad, satt)], dim=2)
        pos = (prefix_pad.sum(-1)[:, None] + torch.cumsum(spad, 1) - 1
               + pos_shift)
        h, _ = O.gemma_model(P, 'llm_expert', cfg.exp_layers, embs, pos, full,
                             cfg, past_kvs=kvs, cond=cond)
        n = cfg.n_action_steps
        out = h[:, :n] if first_rows else h[:, -n:]
        return O.linear(out, P['action_out_proj.projector.weight'],
                        P['action_out_proj.projector.bias'])
    return fn


def test_denoise_step_cached_equals_joint_pass():
    """KV caching must not change the velocity: denoise_step's suffix rows
    over the cached prefix K/V equal the suffix rows of the joint pass,
    whose positions come from the training forward's cumsum over the whole
    pad mask (a different code path of the reference).  A suffix position
    off by one, or the state row kept in the output, breaks it."""
    args = _joint_setup()
    want = _joint_reference(*args)
    got = _cached_velocity(O.denoise_step, *args)
    assert got.shape == want.shape == (2, args[0].n_action_steps, 32)
    assert torch.allclose(got, want, atol=2e-5, rtol=1e-4)
    for bad in (_planted_denoise(pos_shift=-1), _planted_denoise(pos_shift=1),
                _planted_denoise(first_rows=True)):
        assert not torch.allclose(_cached_velocity(bad, *args), want,
                                  atol=1e-3)


def test_product_suffix_positions_follow_joint_cumsum(golden):
    """The kernels' suffix positions (attention_groups) are the suffix part
    of cumsum(joint pad) - 1, the training forward's rule, on the
    reference's own pad fixtures and on a padded prefix."""
    from fluxvla_amd.pi0_inference import attention_groups
    cases = []
    for which in ('pi0', 'pi05'):
        cases.append((torch.from_numpy(golden[f'{which}_prefix_pad_masks']).bool(),
                      torch.from_numpy(golden[f'{which}_suffix_pad_masks']).bool(),
                      torch.from_numpy(golden[f'{which}_suffix_att_masks'])))
    ppad = _joint_setup()[3]
    cases.append((ppad, torch.ones(2, 51, dtype=torch.bool),
                  torch.tensor([[1, 1] + [0] * 49] * 2)))
    for ppad, spad, satt in cases:
        _, _, _, pos_pre, pos_suf = attention_groups(ppad, satt[0].int().tolist())
        joint = torch.cumsum(torch.cat([ppad, spad], 1).long(), 1) - 1
        S = ppad.shape[1]
        assert torch.equal(pos_suf.long(), joint[:, S:])
        valid = ppad
        assert torch.equal(pos_pre.long()[valid], joint[:, :S][valid])


def test_denoise_step_output_rows_closed_form():
    """pi0_flowmatching.py:826-828: v = action_out_proj(final_norm(h))
    over the last n_action_steps rows, i.e. without the state row.  With a
    zero expert the stream is the suffix embedding itself; with the _eye_sd
    projections the action rows are 2 silu(x_t) (zero past dim 32), so
    v = action_out(y * rsqrt(mean(y^2) + eps) * (1 + w)), y = 2 silu(x_t)."""
    cfg = tiny(proj_width=64, exp_hidden=64, exp_mlp=96, heads=2,
               head_dim=16, vit_layers=0, llm_layers=0, exp_layers=1)
    sd = {k: torch.zeros(v.shape) for k, v in
          make_state_dict(cfg, seed=52).items() if k.startswith('llm_expert.')}
    sd.update(_eye_sd(cfg))
    g = torch.Generator().manual_seed(53)
    w_norm = torch.randn(cfg.exp_hidden, generator=g) * 0.1
    sd['llm_expert.norm.weight'] = w_norm
    W = torch.randn(cfg.max_action_dim, cfg.exp_hidden, generator=g) * 0.1
    b = torch.randn(cfg.max_action_dim, generator=g) * 0.1
    sd['action_out_proj.projector.weight'] = W
    sd['action_out_proj.projector.bias'] = b
    B, Sp = 2, 7
    ppad = torch.ones(B, Sp, dtype=torch.bool)
    kvs = [(torch.randn(B, 1, Sp, cfg.head_dim, generator=g),
            torch.randn(B, 1, Sp, cfg.head_dim, generator=g))]
    states = torch.rand(B, cfg.state_dim, generator=g) * 2 - 1
    x_t = torch.randn(B, cfg.n_action_steps, cfg.max_action_dim, generator=g)
    t = torch.tensor([0.6, 0.2])
    y = torch.zeros(B, cfg.n_action_steps, cfg.exp_hidden)
    y[..., :cfg.max_action_dim] = 2 * x_t * torch.sigmoid(x_t)
    n = y / torch.sqrt((y * y).mean(-1, keepdim=True) + cfg.rms_eps)
    want = (n * (1 + w_norm)) @ W.t() + b
    got = O.denoise_step(sd, cfg, states, ppad, kvs, x_t, t)
    assert torch.allclose(got, want, atol=1e-5)
    bad = _planted_denoise(first_rows=True)(sd, cfg, states, ppad, kvs, x_t, t)
    assert not torch.allclose(bad, want, atol=1e-3)


# ---------------------------------------------------------------------------
# guidance with use_vjp (rtc_guidance.py:142-150)
# ---------------------------------------------------------------------------
def test_guidance_vjp_linear_denoiser_closed_form():
    """A linear denoiser v(x) = x A^T + b (per action row) has J_v^T e =
    e A, so the correction is e + (1 - t) e A with e = w (prev - x_1) on the
    previous chunk's rows: the VJP's sign, its (1 - t) factor, the identity
    term and the transposition of A each change the result (A is not
    symmetric)."""
    g = torch.Generator().manual_seed(61)
    B, T, D, L = 2, 50, 32, 30
    x = torch.randn(B, T, D, generator=g)
    prev = torch.randn(B, L, D, generator=g)
    A = torch.randn(D, D, generator=g) / math.sqrt(D)
    b = torch.randn(D, generator=g)
    w = O.compute_prefix_weights(T, 5, 20, 'exp')
    t, gmax = 0.35, 5.0

    def den(z):
        return z @ A.t() + b

    got = O.apply_rtc_guidance(x, den, prev, w, t, gmax, use_vjp=True)
    v = den(x)
    x1 = x + v * (1 - t)
    e = torch.zeros_like(x)
    e[:, :L] = (prev - x1[:, :L]) * w[None, :L, None]
    gw = O.compute_guidance_weight(t, gmax)
    want = v + gw * (e + (1 - t) * e @ A)
    assert torch.allclose(got, want, atol=1e-5)
    for bad in (v + gw * (e - (1 - t) * e @ A), v + gw * (e + e @ A),
                v + gw * (1 - t) * e @ A, v + gw * (e + (1 - t) * e @ A.t())):
        assert not torch.allclose(got, bad, atol=1e-3)
    # without use_vjp the correction is e alone
    plain = O.apply_rtc_guidance(x, den, prev, w, t, gmax)
    assert torch.allclose(plain, v + gw * e, atol=1e-6)


def test_guidance_vjp_constant_velocity_equals_plain_guidance():
    """A denoiser that ignores x has a zero Jacobian: the VJP loop equals
    the loop without it step for step."""
    g = torch.Generator().manual_seed(62)
    B, T, D = 1, 50, 32
    noise = torch.randn(B, T, D, generator=g)
    c = torch.randn(B, T, D, generator=g)
    prev = torch.randn(B, 40, D, generator=g)
    rc = {'method': 'guidance', 'decay_end': 12, 'schedule': 'exp'}
    a = O.euler_guidance_rtc(noise.clone(), lambda x, t: c.clone(), B,
                             torch.tensor(-0.1), prev, 4, rc, T)
    b = O.euler_guidance_rtc(noise.clone(), lambda x, t: c.clone(), B,
                             torch.tensor(-0.1), prev, 4, dict(rc, use_vjp=True),
                             T)
    assert torch.allclose(a, b, atol=1e-6)


@pytest.mark.parametrize('pi05', [False, True])
def test_guidance_vjp_through_denoise_step_finite_differences(pi05):
    """Through the real denoiser (a one-layer expert against a random
    cache): the VJP correction minus e, dotted with a direction d, equals
    -(1 - t) e . J_u d with J_u d from central differences of denoise_step
    (the guidance passes -u as its denoiser)."""
    cfg = tiny(pi05=pi05, proj_width=64, exp_hidden=64, exp_mlp=96, heads=2,
               head_dim=16, vit_layers=0, llm_layers=0, exp_layers=1)
    sd = {k: v.float() for k, v in make_state_dict(cfg, seed=63).items()}
    g = torch.Generator().manual_seed(64)
    B, Sp = 2, 9
    ppad = torch.ones(B, Sp, dtype=torch.bool)
    ppad[1, 6:] = False
    kvs = [(torch.randn(B, 1, Sp, cfg.head_dim, generator=g),
            torch.randn(B, 1, Sp, cfg.head_dim, generator=g))]
    states = torch.rand(B, cfg.state_dim, generator=g) * 2 - 1
    x = torch.randn(B, cfg.n_action_steps, cfg.max_action_dim, generator=g)
    prev = torch.randn(B, 30, cfg.max_action_dim, generator=g)
    w = O.compute_prefix_weights(cfg.n_action_steps, 6, 18, 'linear')
    time = torch.tensor(0.6)

    def u(z):
        return O.denoise_step(sd, cfg, states, ppad, kvs, z, time.expand(B))

    t, gmax = 1.0 - 0.6, 5.0
    with torch.no_grad():
        got = O.apply_rtc_guidance(x, lambda z: -u(z), prev, w, t, gmax,
                                   use_vjp=True)
        plain = O.apply_rtc_guidance(x, lambda z: -u(z), prev, w, t, gmax)
    gw = O.compute_guidance_weight(t, gmax)
    jte_part = (got - plain) / gw  # = -(1 - t) J_u^T e
    v = -u(x)
    e = torch.zeros_like(x)
    e[:, :30] = (prev - (x + v * (1 - t))[:, :30]) * w[None, :30, None]
    for seed in (65, 66):
        d = torch.randn(x.shape, generator=torch.Generator().manual_seed(seed))
        eps = 1e-2
        jd = (u(x + eps * d) - u(x - eps * d)) / (2 * eps)
        lhs = (jte_part * d).sum().item()
        rhs = -(1 - t) * (e * jd).sum().item()
        assert abs(lhs - rhs) <= 2e-3 * abs(rhs) + 1e-5, (lhs, rhs)
        assert abs(rhs) > 1e-2
