"""Host-side logic of the product path, checked on the CPU against the
oracle: weight preparation (norm folds, pair-interleaved Q/K rows, QKV
stacking, patch-weight flattening), the per-step time tables, and the
library's refusal to run without its HIP shared object."""
import pytest
import torch
import torch.nn.functional as F

from fluxvla_amd import pi0_inference as P
from fluxvla_amd.config import tiny
from fluxvla_amd.weights import make_state_dict
from oracle import pi0_oracle as O


@pytest.fixture(scope='module')
def small():
    cfg = tiny(vit_hidden=64, vit_heads=4, vit_layers=1, vit_mlp=96,
               llm_hidden=64, llm_mlp=96, heads=4, head_dim=16, llm_layers=1,
               exp_hidden=32, exp_mlp=48, exp_layers=1, image_size=28,
               patch=14, proj_width=32, max_prompt_len=4)
    sd = {k: v for k, v in make_state_dict(cfg, seed=21).items()}
    return cfg, sd


@pytest.mark.parametrize('role', ['llm', 'expert'])
def test_gemma_prep_equals_norm_then_linear(small, role):
    """x @ qkv_w'^T * rms(x) == [q | k | v](gemma_rms_norm(x)) with Q/K in
    pair-interleaved order; gate/up likewise with the post-attn norm."""
    cfg, sd = small
    W = P.prepare_gemma(sd, cfg, role, 'cpu')
    pre = ('llm_backbone' if role == 'llm' else 'llm_expert') + '.layers.0'
    hid = cfg.llm_hidden if role == 'llm' else cfg.exp_hidden
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, hid, generator=g)
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.rms_eps)
    L = W['layers'][0]
    got = (x @ L['qkv_w'].float().t()) * r
    xn = O.gemma_rms_norm(x, sd[f'{pre}.input_layernorm.weight'], cfg.rms_eps)
    q = O.linear(xn, sd[f'{pre}.self_attn.q_proj.weight'])
    k = O.linear(xn, sd[f'{pre}.self_attn.k_proj.weight'])
    v = O.linear(xn, sd[f'{pre}.self_attn.v_proj.weight'])
    perm = P.interleave_rows(cfg.head_dim)
    q = q.view(5, cfg.heads, cfg.head_dim)[:, :, perm].reshape(5, -1)
    want = torch.cat([q, k[:, perm], v], 1)
    assert torch.allclose(got, want, atol=2e-2 * want.abs().max().item())
    xn2 = O.gemma_rms_norm(x, sd[f'{pre}.post_attention_layernorm.weight'],
                           cfg.rms_eps)
    got_g = (x @ L['gate_w'].float().t()) * r
    want_g = O.linear(xn2, sd[f'{pre}.mlp.gate_proj.weight'])
    assert torch.allclose(got_g, want_g, atol=2e-2 * want_g.abs().max().item())


def test_final_norm_fold_into_action_out(small):
    cfg, sd = small
    W = P.prepare_gemma(sd, cfg, 'expert', 'cpu')
    w_out = (sd['action_out_proj.projector.weight'].float() *
             W['final_scale'][None])
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, cfg.exp_hidden, generator=g)
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.rms_eps)
    got = (x @ w_out.t()) * r
    want = O.linear(O.gemma_rms_norm(x, sd['llm_expert.norm.weight'],
                                     cfg.rms_eps),
                    sd['action_out_proj.projector.weight'])
    assert torch.allclose(got, want, atol=1e-4)


def test_siglip_patch_weight_order(small):
    """im2col column order (c, ky, kx) against conv2d."""
    cfg, sd = small
    V = P.prepare_siglip(sd, cfg, 'cpu')
    g = torch.Generator().manual_seed(3)
    img = torch.rand(2, 3, 28, 28, generator=g)
    p = cfg.patch
    cols = F.unfold(img, p, stride=p).transpose(1, 2)  # (c, ky, kx) order
    cols = F.pad(cols, (0, cfg.patch_k_pad - cfg.patch_k))
    got = cols @ V['patch_w'].float().t() + V['patch_b'].float()
    w = sd[f'{P.VIS}.embeddings.patch_embedding.weight'].float()
    ref = F.conv2d(img, w, V['patch_b'].float(), stride=p)
    ref = ref.flatten(2).transpose(1, 2)
    assert torch.allclose(got, ref, atol=1e-4)
    L = V['layers'][0]
    assert L['qkv_w'].shape == (3 * cfg.vit_hidden, cfg.vit_hidden)


def test_time_tables_match_oracle():
    ts, dt = P.euler_times(10)
    assert ts == O.euler_times(10)
    assert dt == float(torch.tensor(-0.1, dtype=torch.float32))
    emb = P.sinusoid(ts, 64)
    ref = O.sinusoidal_pos_embedding(torch.tensor(ts), 64, 4e-3, 4.0)
    assert torch.equal(emb, ref)


def test_kv_len_is_vector_aligned():
    cfg = tiny()
    obj = P.PI0Inference.__new__(P.PI0Inference)
    obj.cfg = cfg
    assert obj.kv_len % 8 == 0 and obj.kv_len >= cfg.prefix_len + cfg.suffix_len


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from fluxvla_amd import _lib
    monkeypatch.setattr(_lib, 'LIB_PATH', str(tmp_path / 'absent.so'))
    monkeypatch.setattr(_lib, '_lib', None)
    with pytest.raises(ImportError, match='not built'):
        _lib.load()


def _reference_style_cfg(type_name, pi05):
    """A model dict shaped like the reference's PI0 / PI0.5 configs (the
    keys build_vla_from_cfg reads), with the PI0 dimensions."""
    gemma = dict(type='ConditionGemmaModel', head_dim=256, hidden_size=2048,
                 intermediate_size=16384, num_attention_heads=8,
                 num_hidden_layers=18, num_key_value_heads=1,
                 rms_norm_eps=1e-06, rope_theta=10000.0, vocab_size=257152)
    expert = dict(gemma, hidden_size=1024, intermediate_size=4096,
                  use_adarms=pi05, adarms_cond_dim=1024 if pi05 else None)
    cfg = dict(type=type_name, llm_backbone=gemma, llm_expert=expert,
               vision_backbone=dict(
                   type='SigLIPViTBackbone', vision_backbone_id='siglip_224',
                   vision_config=dict(hidden_size=1152, image_size=224,
                                      intermediate_size=4304,
                                      layer_norm_eps=1e-06,
                                      num_attention_heads=16,
                                      num_hidden_layers=27, patch_size=14)),
               proj_width=1024, n_action_steps=50, max_action_dim=32)
    if not pi05:
        cfg['state_proj'] = dict(type='LinearProjector', in_dim=32,
                                 out_dim=1024)
    return cfg


@pytest.mark.parametrize('name,pi05', [('PI0FlowMatching', False),
                                       ('PI05FlowMatchingInference', True)])
def test_registry_reads_reference_configs(name, pi05):
    from fluxvla_amd.config import PI0Config
    from fluxvla_amd.registry import VLAS, config_from_reference
    cfg = config_from_reference(_reference_style_cfg(name, pi05), num_views=3)
    assert name in VLAS
    assert cfg == PI0Config(pi05=pi05)


def test_registry_rejects_unknown_type():
    from fluxvla_amd.registry import build_vla_from_cfg
    with pytest.raises(KeyError, match='not a registered'):
        build_vla_from_cfg(dict(type='OpenVLA'))


def test_fragment_major_layouts():
    """FragA / FragB packing puts element (r, c) where the kernels'
    frag_offset formula says: ((c/32 * 4 + r/16) * 64 + (c%32)/8 * 16 +
    r%16) * 8 + c%8 for A, and the same with the 16-row tile index leading
    for B."""
    import torch
    from fluxvla_amd import kernels as K
    m, k = 37, 96
    a = torch.arange(m * k, dtype=torch.float32).view(m, k)
    pa = K.pack_frag_a_ref(a)
    for r, c in [(0, 0), (5, 9), (16, 31), (36, 95), (20, 40)]:
        off = ((c // 32 * 4 + r // 16) * 64 + (c % 32) // 8 * 16 + r % 16) * 8 + c % 8
        assert pa[off].item() == a[r, c].item()
    n = 48
    w = torch.arange(n * k, dtype=torch.float32).view(n, k)
    pb = K.FragB.pack(w).buf
    for r, c in [(0, 0), (5, 9), (16, 31), (47, 95), (33, 70)]:
        off = (((r // 16) * (k // 32) + c // 32) * 64 + (c % 32) // 8 * 16 +
               r % 16) * 8 + c % 8
        assert pb[off].item() == w[r, c].item()


# ---------------------------------------------------------------------------
# Real-time chunking host tables (fluxvla_amd/rtc.py) against the oracle
# ---------------------------------------------------------------------------
@pytest.mark.parametrize('schedule', ['exp', 'linear', 'ones', 'zeros'])
@pytest.mark.parametrize('prefix_len,decay_end', [(5, 10), (0, 10), (48, 60),
                                                  (7, 7), (3, 4)])
def test_rtc_prefix_weights_match_oracle(schedule, prefix_len, decay_end):
    from fluxvla_amd import rtc as R
    assert torch.equal(
        R.compute_prefix_weights(50, prefix_len, decay_end, schedule),
        O.compute_prefix_weights(50, prefix_len, decay_end, schedule))


def test_rtc_guidance_cw_matches_oracle_update():
    """One guidance step through the fused update x + dt v + cw (prev - x +
    omt v) equals the oracle's apply_rtc_guidance step at every step."""
    from fluxvla_amd import rtc as R
    g = torch.Generator().manual_seed(3)
    times, dt = P.euler_times(10)
    rc = {'max_guidance_weight': 4.0, 'decay_end': 16, 'schedule': 'exp'}
    L = 30
    cw = R.guidance_cw(times, dt, 50, 6, L, rc)
    omt = R.guidance_omt(times)
    w = O.compute_prefix_weights(50, 6, 16, 'exp')
    x = torch.randn(1, 50, 32, generator=g)
    v = torch.randn(1, 50, 32, generator=g)
    prev = torch.randn(1, L, 32, generator=g)
    prev_pad = torch.zeros(1, 50, 32)
    prev_pad[:, :L] = prev
    for k, time in enumerate(times):
        v_fm = O.apply_rtc_guidance(x, lambda z: -v, prev, w, 1.0 - time, 4.0)
        ref = x + dt * (-v_fm)
        got = x + dt * v + cw[k][None, :, None] * (prev_pad - x + omt[k] * v)
        assert torch.allclose(got, ref, atol=1e-5), k
    assert torch.equal(cw[:, L:], torch.zeros(10, 50 - L))


def test_rtc_method_selection_and_padding():
    from fluxvla_amd import rtc as R
    prev = torch.ones(1, 5, 14)
    assert R.select_method(prev, 3, {'enabled': True}) == 'prefix'
    assert R.select_method(prev, 3, {'method': 'guidance'}) == 'guidance'
    assert R.select_method(prev, 0, {'method': 'prefix'}) is None
    assert R.select_method(None, 3, {'method': 'prefix'}) is None
    assert R.select_method(prev, 3, None) is None
    assert R.select_method(prev, 3, {'method': 'other'}) is None
    assert R.select_method(prev, 3, {'method': 'guidance',
                                     'use_vjp': True}) == 'guidance_vjp'
    assert R.select_method(prev, 3, {'method': 'guidance',
                                     'use_vjp': False}) == 'guidance'
    p = R.pad_prev_actions(prev, 32, 14)
    assert p.shape == (1, 5, 32) and torch.equal(p[..., 14:],
                                                 torch.zeros(1, 5, 18))
    with pytest.raises(ValueError):
        R.pad_prev_actions(prev, 32, None)


def test_rtc_guidance_vjp_tables_match_oracle():
    """The VJP update's device tables: the oracle's prefix weights with the
    rows past the previous chunk zeroed, and the oracle's guidance weight at
    t = 1 - time of each step."""
    from fluxvla_amd import rtc as R
    from fluxvla_amd.pi0_inference import euler_times
    from oracle import pi0_oracle as O
    times, _ = euler_times(10)
    rc = {'decay_end': 17, 'schedule': 'linear', 'max_guidance_weight': 3.0}
    w, gw = R.guidance_vjp_tables(times, 50, 6, 24, rc)
    want = O.compute_prefix_weights(50, 6, 17, 'linear')
    want[24:] = 0
    assert torch.allclose(w, want)
    assert gw.shape == (10,)
    for k, time in enumerate(times):
        assert abs(gw[k].item() - O.compute_guidance_weight(1.0 - time, 3.0)) < 1e-6
    assert gw[0].item() == 3.0  # capped at pure noise
