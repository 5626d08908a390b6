"""The fluxvla/ops/atomic_ops.py mirror, called the way the reference's fused
model calls it (pi05_flowmatching_inference.py:22-66 vision layer,
:187-286 expert layer), with weights from the matching prepare hooks,
checked against the CPU oracle.  Real widths, one layer."""
import pytest
import torch

from fluxvla_amd import atomic_ops as A
from fluxvla_amd import kernels as Kn
from fluxvla_amd import pi0_inference as P
from fluxvla_amd.config import tiny
from fluxvla_amd.weights import make_state_dict
from oracle import pi0_oracle as O
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def rel_err(out, ref):
    out, ref = out.detach().float().cpu(), ref.detach().float().cpu()
    return ((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def test_siglip_layer_via_atomic_ops(cuda):
    announce('atomic_ops siglip layer (vision_encoder call order)')
    cfg = tiny(vit_layers=1, llm_layers=0, exp_layers=0)
    sd = make_state_dict(cfg, seed=31)
    V = P.prepare_siglip(sd, cfg, cuda)
    nv, np_, vh = 3, cfg.num_patches, cfg.vit_hidden
    g = torch.Generator().manual_seed(32)
    imgs = torch.rand(nv, 3, 224, 224, generator=g) * 2 - 1
    nhwc = imgs.permute(0, 2, 3, 1).contiguous().bfloat16().to(cuda)
    bf = dict(dtype=torch.bfloat16, device=cuda)
    x = torch.empty(nv, np_, vh, **bf)
    xn = torch.empty_like(x)
    qkv = torch.empty(nv, np_, 3 * vh, **bf)
    hid = torch.empty(nv, np_, cfg.vit_mlp, **bf)
    A.conv2d_embed_res(nhwc, V['patch_w'], V['patch_b'], V['pos_emb'], x, 16,
                       14, np_, vh)
    L = V['layers'][0]
    A.layer_norm_QKV_matmul_bias(x, L['ln1_w'], L['ln1_b'], L['qkv_w'],
                                 L['qkv_b'], qkv, xn, np_, vh, 3 * vh)
    attn = A.AttnMultiKey(qkv, np_, cfg.vit_heads, cfg.vit_head_dim, vh)
    A.matmul_bias_res(attn, L['o_w'], L['o_b'], x, x, None, np_, vh)
    A.layer_norm_matmul_bias_gelu(x, L['ln2_w'], L['ln2_b'], L['fc1_w'],
                                  L['fc1_b'], hid, xn, np_, vh, cfg.vit_mlp)
    A.matmul_split_k_bias_res(hid, L['fc2_w'], L['fc2_b'], x, x, None, np_,
                              cfg.vit_mlp, vh)
    out = Kn.layer_norm(x.view(-1, vh), V['post_ln_w'], V['post_ln_b'], 1e-6)
    ref = O.siglip_tower(sd, imgs.bfloat16().float(), cfg).reshape(-1, vh)
    assert rel_err(out, ref) <= 1e-2


def reference_rope_table(positions, head_dim, theta=10000.0):
    """The reference fast path's table: interleaved (cos, sin) pairs in bf16
    per position (pi05_flowmatching_inference.py:444-456)."""
    inv = 1.0 / (theta**(torch.arange(0, head_dim, 2).float() / head_dim))
    ph = positions.float()[:, None] * inv[None, :]
    return torch.stack([ph.cos(), ph.sin()], -1).to(
        torch.bfloat16).reshape(len(positions), head_dim)


def test_pi05_expert_layer_via_atomic_ops(cuda):
    """adaRMS expert layer on 50 tokens, self-attention only, in the
    reference's op order; vs the oracle's GemmaDecoderLayer with cond."""
    announce('atomic_ops pi05 expert layer (transformer_decoder call order)')
    cfg = tiny(pi05=True, vit_layers=0, llm_layers=1, exp_layers=1)
    sd = make_state_dict(cfg, seed=33)
    E = P.prepare_gemma(sd, cfg, 'expert', cuda)
    L = E['layers'][0]
    S, hid, D, H = 50, cfg.exp_hidden, cfg.head_dim, cfg.heads
    g = torch.Generator().manual_seed(34)
    x0 = torch.randn(S, hid, generator=g).bfloat16()
    cond = torch.randn(1, cfg.proj_width, generator=g).bfloat16()
    bf = dict(dtype=torch.bfloat16, device=cuda)
    x = x0.to(cuda)
    temb = cond.to(cuda).expand(S, -1).contiguous()
    xn, gate = torch.empty(S, hid, **bf), torch.empty(S, hid, **bf)
    style = torch.empty(S, 3 * hid, **bf)
    q = torch.empty(S, H * D, **bf)
    k, v = torch.empty(S, D, **bf), torch.empty(S, D, **bf)
    ctx = torch.empty(S, H * D, **bf)
    h = torch.empty(S, cfg.exp_mlp, **bf)
    rope = reference_rope_table(torch.arange(S), D).to(cuda)
    A.adarms_norm_style_proj(x, temb, L['attn_mod_w'], L['attn_mod_b'], xn,
                             gate, style, hid, 3 * hid)
    A.matmul_qkv_rope(xn, L['qkv_w'], rope, q, k, v, hid, D, H)
    Kn.mqa_attention(q.view(1, S, H, D), k.view(1, S, D), v.view(1, S, D),
                     ctx.view(1, S, H, D))
    A.matmul_res_gate(ctx, L['o_w'], x, gate, H * D, hid)
    A.adarms_norm_style_proj(x, temb, L['ffn_mod_w'], L['ffn_mod_b'], xn,
                             gate, style, hid, 3 * hid)
    A.matmul_gate(xn, L['gate_w'], L['up_w'], h, hid, cfg.exp_mlp)
    A.matmul_res_gate(h, L['down_w'], x, gate, cfg.exp_mlp, hid)
    pos = torch.arange(S)[None]
    cos, sin = O.rope_cos_sin(pos, D, cfg.rope_theta)
    ref, _ = O.gemma_layer(sd, 'llm_expert.layers.0', x0.float()[None], cos,
                           sin, None, None, cond.float(), cfg)
    assert rel_err(x, ref[0]) <= 1e-2


@pytest.mark.parametrize('layout', ['nk', 'kn'])
def test_matmul_bias_cuda(cuda, layout):
    announce(f'matmul_bias_cuda layout={layout}')
    g = torch.Generator().manual_seed(35)
    inp = torch.randn(3, 256, 1152, generator=g).bfloat16()
    w = (torch.randn(1152, 1152, generator=g) * 0.02).bfloat16()  # [N, K]
    b = (torch.randn(1152, generator=g) * 0.1).bfloat16()
    res = torch.randn(3, 256, 1152, generator=g).bfloat16()
    wd = (w if layout == 'nk' else w.t().contiguous()).to(cuda)
    out = A.matmul_bias_cuda(inp.to(cuda), wd, b.to(cuda), res=res.to(cuda),
                             weight_layout=layout)
    ref = inp.float() @ w.float().t() + b.float() + res.float()
    assert out.shape == (3, 256, 1152)
    assert rel_err(out, ref) <= 1e-2
    bad = wd[:, :100] if layout == 'nk' else wd[:100]  # wrong K
    with pytest.raises(ValueError):
        A.matmul_bias_cuda(inp.to(cuda), bad.contiguous(), b.to(cuda),
                           weight_layout=layout)
