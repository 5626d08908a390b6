"""CPU oracle of the PI0 / PI0.5 inference path (fp32 PyTorch on the CPU).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module, and only as the checker
(or the timed CPU baseline) -- never as the thing measured or shipped.  The
product path (fluxvla_amd/) runs the HIP kernels and fails loudly without
them.

It restates the reference's eager PyTorch path, which the reference itself
uses as PI0's only inference path (BaseVLA -> PI0FlowMatching.predict_action):

  predict_action   fluxvla/models/vlas/pi0_flowmatching.py:702-785, 642-649
  RTC loops        pi0_flowmatching.py:651-700,
                   fluxvla/engines/utils/rtc_guidance.py:28-155 (the VJP
                   of use_vjp by torch autograd, as the reference)
  embed_prefix     pi0_flowmatching.py:204-250
  embed_suffix     pi0_flowmatching.py:252-321 (PI0),
                   fluxvla/models/vlas/pi05_flowmatching.py:68-127 (PI0.5)
  denoise_step     pi0_flowmatching.py:787-831
  Gemma model      fluxvla/models/backbones/llms/condition_gemma.py:45-147
                   (GemmaRMSNorm), 156-192 (GemmaMLP), 195-299 (RoPE),
                   340-535 (attention), 561-662 (decoder layer), 833-994
  masks / time     fluxvla/engines/utils/model_utils.py:40-95
  SigLIP tower     HF SiglipVisionModel (transformers, third party) as
                   configured by configs/pi0/pi0_paligemma_aloha_full_
                   finetune.py:41-61, called per view and concatenated
                   (fluxvla/models/backbones/visions/siglip_vit.py:107-126)

Everything runs in fp32 from the bf16 parameters (upcast once), i.e. the
exact math of the reference path without its bf16 activation rounding.

How each part is pinned (tests/test_oracle.py): library routines (torch's
gelu(tanh), layer_norm, scaled_dot_product_attention, conv2d; the HF
transformers Gemma and SigLIP modules installed here), invariants (RoPE
relative-position property and norm preservation; permutation of Q/K rows;
softmax rows sum to one and masked keys weigh zero; split-KV merge), the
reference's own mask fixtures (test/data/models/vlas/pi0{,5}/*_masks.npy
copied to tests/golden/), and closed forms (Euler loop with one step,
zeroed expert).
"""
import math

import torch
import torch.nn.functional as F

BF16_MIN = float(torch.finfo(torch.bfloat16).min)
VIS = 'vision_backbone.vision.vision_model'


def _f(t):
    return t.float()


def linear(x, w, b=None):
    """nn.Linear: x @ w^T + b."""
    return F.linear(x, _f(w), None if b is None else _f(b))


def gemma_rms_norm(x, w, eps):
    """GemmaRMSNorm, plain mode (condition_gemma.py:75-80, 113-116):
    x * rsqrt(mean(x^2) + eps) * (1 + w)."""
    var = torch.mean(torch.square(x), dim=-1, keepdim=True)
    return x * torch.rsqrt(var + eps) * (1.0 + _f(w))


def ada_rms_norm(x, cond, dense_w, dense_b, eps):
    """GemmaRMSNorm, adaptive mode (condition_gemma.py:118-147):
    [scale, shift, gate] = dense(cond); rms(x) * (1 + scale) + shift.
    Returns (normed, gate)."""
    mod = linear(cond, dense_w, dense_b)
    if mod.dim() == 2 and x.dim() == 3:
        mod = mod[:, None]
    scale, shift, gate = torch.chunk(mod, 3, dim=-1)
    var = torch.mean(torch.square(x), dim=-1, keepdim=True)
    n = x * torch.rsqrt(var + eps)
    return n * (1 + scale) + shift, gate


def gelu_tanh(x):
    """ACT2FN['gelu_pytorch_tanh'] (condition_gemma.py:175, hidden_act)."""
    return F.gelu(x, approximate='tanh')


def rope_cos_sin(position_ids, head_dim, theta):
    """GemmaRotaryEmbedding.forward with the default rope init
    (condition_gemma.py:216-260): inv_freq = 1 / theta^(2i/d) in fp32,
    freqs = pos * inv_freq, emb = cat(freqs, freqs)."""
    inv = 1.0 / (theta**(torch.arange(0, head_dim, 2, dtype=torch.int64)
                         .float() / head_dim))
    freqs = position_ids[..., None].float() * inv
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x):
    """condition_gemma.py:263-267."""
    x1 = x[..., :x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(q, k, cos, sin):
    """apply_rotary_pos_emb with unsqueeze_dim=1 (condition_gemma.py:270-299)."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def attention(q, k, v, mask, scaling):
    """eager_attention_forward (condition_gemma.py:340-365) for one shared
    K/V head (repeat_kv), with the reference's additive bf16-min mask
    (pi0_flowmatching.py:522-527).  q [B, H, Sq, D]; k, v [B, 1, Sk, D];
    mask bool [B, Sq, Sk] (True = visible) or None."""
    k = k.expand(-1, q.shape[1], -1, -1)
    v = v.expand(-1, q.shape[1], -1, -1)
    w = torch.matmul(q, k.transpose(2, 3)) * scaling
    if mask is not None:
        add = torch.zeros(mask.shape, dtype=torch.float32)
        add.masked_fill_(~mask, BF16_MIN)
        w = w + add[:, None]
    w = torch.softmax(w, dim=-1, dtype=torch.float32)
    return torch.matmul(w, v)


def make_att_2d_masks(pad_masks, att_masks):
    """model_utils.py:77-95: visible iff cumsum(att)[j] <= cumsum(att)[i]
    and both tokens are valid."""
    cumsum = torch.cumsum(att_masks, dim=1)
    att_2d = cumsum[:, None, :] <= cumsum[:, :, None]
    pad_2d = pad_masks[:, None, :] * pad_masks[:, :, None]
    return att_2d & pad_2d


def sinusoidal_pos_embedding(time, dimension, min_period, max_period):
    """create_sinusoidal_pos_embedding (model_utils.py:40-68), fp32."""
    fraction = torch.linspace(0.0, 1.0, dimension // 2, dtype=torch.float32)
    period = min_period * (max_period / min_period)**fraction
    scaling_factor = 1.0 / period * 2 * math.pi
    sin_input = time[..., None] * scaling_factor
    return torch.cat([torch.sin(sin_input), torch.cos(sin_input)], dim=-1)


def euler_times(num_steps):
    """The fp32 time values the Euler loop visits
    (pi0_flowmatching.py:642-649): time = 1; while time >= -dt/2: ...;
    time += dt, all in fp32."""
    dt = torch.tensor(-1.0 / num_steps, dtype=torch.float32)
    time = torch.tensor(1.0, dtype=torch.float32)
    out = []
    while time >= -dt / 2:
        out.append(float(time))
        time = time + dt
    return out


# ---------------------------------------------------------------------------
# Gemma (ConditionGemmaModel)
# ---------------------------------------------------------------------------
def gemma_layer(P, pre, h, cos, sin, mask, past_kv, cond, cfg,
                kv_only=False):
    """GemmaDecoderLayer.forward (condition_gemma.py:561-662) with
    GemmaAttention (:468-535).  Returns (h, (k, v)) where k, v are this
    layer's post-RoPE key/value states [B, 1, S, D] (what the prefix cache
    stores, :500-509)."""
    B, S, _ = h.shape
    H, D, eps = cfg.heads, cfg.head_dim, cfg.rms_eps
    resid = h
    if cond is None:
        x, gate = gemma_rms_norm(h, P[f'{pre}.input_layernorm.weight'],
                                 eps), None
    else:
        x, gate = ada_rms_norm(h, cond, P[f'{pre}.input_layernorm.dense.weight'],
                               P[f'{pre}.input_layernorm.dense.bias'], eps)
    q = linear(x, P[f'{pre}.self_attn.q_proj.weight']).view(B, S, H,
                                                            D).transpose(1, 2)
    k = linear(x, P[f'{pre}.self_attn.k_proj.weight']).view(B, S, 1,
                                                            D).transpose(1, 2)
    v = linear(x, P[f'{pre}.self_attn.v_proj.weight']).view(B, S, 1,
                                                            D).transpose(1, 2)
    q, k = apply_rope(q, k, cos, sin)
    if kv_only:
        return None, (k, v)
    if past_kv is not None:
        kk = torch.cat([past_kv[0], k], dim=2)
        vv = torch.cat([past_kv[1], v], dim=2)
    else:
        kk, vv = k, v
    o = attention(q, kk, vv, mask, D**-0.5)
    o = o.transpose(1, 2).reshape(B, S, H * D)
    o = linear(o, P[f'{pre}.self_attn.o_proj.weight'])
    h = resid + (o if gate is None else o * gate)
    resid = h
    if cond is None:
        x, gate = gemma_rms_norm(
            h, P[f'{pre}.post_attention_layernorm.weight'], eps), None
    else:
        x, gate = ada_rms_norm(
            h, cond, P[f'{pre}.post_attention_layernorm.dense.weight'],
            P[f'{pre}.post_attention_layernorm.dense.bias'], eps)
    m = linear(
        gelu_tanh(linear(x, P[f'{pre}.mlp.gate_proj.weight'])) *
        linear(x, P[f'{pre}.mlp.up_proj.weight']),
        P[f'{pre}.mlp.down_proj.weight'])
    h = resid + (m if gate is None else m * gate)
    return h, (k, v)


def gemma_model(P, prefix, n_layers, h, position_ids, mask, cfg,
                past_kvs=None, cond=None, kv_only_last=False):
    """ConditionGemmaModel.forward (condition_gemma.py:833-994): layers then
    the final norm.  With kv_only_last the last layer stops after its K/V
    (its attention output and MLP only feed the unused prefix hidden state)
    and no final norm is applied."""
    cos, sin = rope_cos_sin(position_ids, cfg.head_dim, cfg.rope_theta)
    kvs = []
    for i in range(n_layers):
        last = kv_only_last and i == n_layers - 1
        hn, kv = gemma_layer(P, f'{prefix}.layers.{i}', h, cos, sin, mask,
                             None if past_kvs is None else past_kvs[i], cond,
                             cfg, kv_only=last)
        kvs.append(kv)
        if not last:
            h = hn
    if kv_only_last:
        return None, kvs
    if cond is None:
        h = gemma_rms_norm(h, P[f'{prefix}.norm.weight'], cfg.rms_eps)
    else:
        h, _ = ada_rms_norm(h, cond, P[f'{prefix}.norm.dense.weight'],
                            P[f'{prefix}.norm.dense.bias'], cfg.rms_eps)
    return h, kvs


# ---------------------------------------------------------------------------
# SigLIP vision tower (HF SiglipVisionModel semantics)
# ---------------------------------------------------------------------------
def siglip_tower(P, pixels, cfg):
    """pixels [N, 3, H, W] -> last_hidden_state [N, patches, vit_hidden]:
    patch conv + position embedding, pre-LN encoder layers (LayerNorm eps
    from the config, bidirectional softmax attention with scale
    head_dim^-0.5, gelu_tanh MLP), post LayerNorm; no pooling head
    (vision_use_head=False)."""
    vh, nh = cfg.vit_hidden, cfg.vit_heads
    hd = vh // nh
    eps = cfg.vit_eps
    x = F.conv2d(pixels, _f(P[f'{VIS}.embeddings.patch_embedding.weight']),
                 _f(P[f'{VIS}.embeddings.patch_embedding.bias']),
                 stride=cfg.patch)
    x = x.flatten(2).transpose(1, 2)
    x = x + _f(P[f'{VIS}.embeddings.position_embedding.weight'])[None]
    N, S, _ = x.shape
    for i in range(cfg.vit_layers):
        pre = f'{VIS}.encoder.layers.{i}'
        r = x
        y = F.layer_norm(x, (vh, ), _f(P[f'{pre}.layer_norm1.weight']),
                         _f(P[f'{pre}.layer_norm1.bias']), eps)

        def proj(nm, t):
            return linear(t, P[f'{pre}.self_attn.{nm}.weight'],
                          P[f'{pre}.self_attn.{nm}.bias'])

        q = proj('q_proj', y).view(N, S, nh, hd).transpose(1, 2)
        k = proj('k_proj', y).view(N, S, nh, hd).transpose(1, 2)
        v = proj('v_proj', y).view(N, S, nh, hd).transpose(1, 2)
        w = torch.softmax(torch.matmul(q, k.transpose(2, 3)) * hd**-0.5,
                          dim=-1, dtype=torch.float32)
        a = torch.matmul(w, v).transpose(1, 2).reshape(N, S, vh)
        x = r + proj('out_proj', a)
        r = x
        y = F.layer_norm(x, (vh, ), _f(P[f'{pre}.layer_norm2.weight']),
                         _f(P[f'{pre}.layer_norm2.bias']), eps)
        y = linear(
            gelu_tanh(linear(y, P[f'{pre}.mlp.fc1.weight'],
                             P[f'{pre}.mlp.fc1.bias'])),
            P[f'{pre}.mlp.fc2.weight'], P[f'{pre}.mlp.fc2.bias'])
        x = r + y
    return F.layer_norm(x, (vh, ), _f(P[f'{VIS}.post_layernorm.weight']),
                        _f(P[f'{VIS}.post_layernorm.bias']), eps)


# ---------------------------------------------------------------------------
# PI0 / PI0.5
# ---------------------------------------------------------------------------
def embed_prefix(P, cfg, images, lang_tokens, img_masks, lang_masks):
    """pi0_flowmatching.py:204-250: SigLIP per view (siglip_vit.py:119-126),
    projector, language embeddings * sqrt(width); prefix attention is
    bidirectional (att mask all 0)."""
    B = images.shape[0]
    pix = images.float().unflatten(1, (-1, 3))
    toks = [siglip_tower(P, pix[:, i], cfg) for i in range(pix.shape[1])]
    img_emb = linear(torch.cat(toks, dim=1), P['projector.projector.weight'],
                     P['projector.projector.bias'])
    n_img = img_emb.shape[1] // img_masks.shape[1]
    pads = [img_masks[:, i:i + 1].expand(B, n_img)
            for i in range(img_masks.shape[1])]
    lang_emb = _f(P['llm_backbone.embed_tokens.weight'])[lang_tokens]
    lang_emb = lang_emb * math.sqrt(lang_emb.shape[-1])
    embs = torch.cat([img_emb, lang_emb], dim=1)
    pad = torch.cat(pads + [lang_masks.bool()], dim=1)
    att = torch.zeros(B, embs.shape[1], dtype=torch.bool)
    return embs, pad, att


def embed_suffix(P, cfg, states, x_t, timestep):
    """PI0 (pi0_flowmatching.py:252-321) or PI0.5
    (pi05_flowmatching.py:68-127).  Returns (embs, pad, att, adarms_cond)."""
    B = x_t.shape[0]
    n = cfg.n_action_steps
    time_emb = sinusoidal_pos_embedding(timestep, cfg.proj_width, 4e-3, 4.0)
    action_emb = linear(x_t, P['action_in_proj.projector.weight'],
                        P['action_in_proj.projector.bias'])
    if cfg.pi05:
        te = F.silu(linear(time_emb, P['time_mlp_in.projector.weight'],
                           P['time_mlp_in.projector.bias']))
        te = F.silu(linear(te, P['time_mlp_out.projector.weight'],
                           P['time_mlp_out.projector.bias']))
        att = torch.tensor([1] + [0] * (n - 1), dtype=torch.bool)
        pad = torch.ones(B, n, dtype=torch.bool)
        return action_emb, pad, att[None].expand(B, n), te
    state_emb = linear(states, P['state_proj.projector.weight'],
                       P['state_proj.projector.bias'])
    if time_emb.dim() == 2:
        time_emb = time_emb[:, None, :].expand_as(action_emb)
    at = torch.cat([action_emb, time_emb], dim=2)
    at = linear(at, P['action_time_mlp_in.projector.weight'],
                P['action_time_mlp_in.projector.bias'])
    at = F.silu(at)
    at = linear(at, P['action_time_mlp_out.projector.weight'],
                P['action_time_mlp_out.projector.bias'])
    embs = torch.cat([state_emb[:, None, :], at], dim=1)
    att = torch.tensor([1, 1] + [0] * (n - 1), dtype=torch.bool)
    pad = torch.ones(B, n + 1, dtype=torch.bool)
    return embs, pad, att[None].expand(B, n + 1), None


def prefix_forward(P, cfg, images, lang_tokens, img_masks, lang_masks):
    """Prefix pass of predict_action (pi0_flowmatching.py:722-742): returns
    (per-layer (k, v) cache, prefix pad mask)."""
    embs, pad, att = embed_prefix(P, cfg, images, lang_tokens, img_masks,
                                  lang_masks)
    mask = make_att_2d_masks(pad, att)
    pos = torch.cumsum(pad, dim=1) - 1
    _, kvs = gemma_model(P, 'llm_backbone', cfg.llm_layers, embs, pos, mask,
                         cfg, kv_only_last=True)
    return kvs, pad


def denoise_step(P, cfg, states, prefix_pad, kvs, x_t, timestep):
    """pi0_flowmatching.py:787-831: velocity v_t [B, n_action_steps, 32]."""
    embs, spad, satt, cond = embed_suffix(P, cfg, states, x_t, timestep)
    B, Ss = spad.shape
    Sp = prefix_pad.shape[1]
    prefix_2d = prefix_pad[:, None, :].expand(B, Ss, Sp)
    suffix_2d = make_att_2d_masks(spad, satt)
    full = torch.cat([prefix_2d, suffix_2d], dim=2)
    pos = torch.sum(prefix_pad, dim=-1)[:, None] + torch.cumsum(spad, 1) - 1
    h, _ = gemma_model(P, 'llm_expert', cfg.exp_layers, embs, pos, full, cfg,
                       past_kvs=kvs, cond=cond)
    out = h[:, -cfg.n_action_steps:]
    return linear(out, P['action_out_proj.projector.weight'],
                  P['action_out_proj.projector.bias'])


# ---------------------------------------------------------------------------
# Euler loops: plain and real-time chunking (RTC)
# ---------------------------------------------------------------------------
def euler_plain(x_t, denoise, bsize, dt):
    """_predict_action_plain (pi0_flowmatching.py:642-649)."""
    time = torch.tensor(1.0, dtype=torch.float32)
    while time >= -dt / 2:
        v_t = denoise(x_t, time.expand(bsize))
        x_t += dt * v_t
        time += dt
    return x_t


def euler_prefix_rtc(x_t, denoise, bsize, dt, prev_actions, prefix_len,
                     n_action_steps):
    """_predict_action_prefix_rtc (pi0_flowmatching.py:651-669): the first
    prefix_len positions are overwritten with the previous chunk before
    every denoise call and at the end, and are denoised at time 0 (clean)."""
    time = torch.tensor(1.0, dtype=torch.float32)
    prefix_mask = torch.zeros(bsize, n_action_steps, dtype=torch.bool)
    prefix_mask[:, :prefix_len] = True
    while time >= -dt / 2:
        t_batch = time.expand(bsize)
        x_t[:, :prefix_len] = prev_actions[:, :prefix_len]
        t_pos = t_batch.unsqueeze(1).expand(-1, n_action_steps).clone()
        t_pos[prefix_mask] = 0.0
        v_t = denoise(x_t, t_pos)
        x_t += dt * v_t
        time += dt
    x_t[:, :prefix_len] = prev_actions[:, :prefix_len]
    return x_t


def compute_prefix_weights(n_action_steps, prefix_len, decay_end,
                           schedule='exp'):
    """compute_prefix_weights (fluxvla/engines/utils/rtc_guidance.py:28-80):
    1 on the locked prefix, then a decay to decay_end ('exp': exp(-3 f),
    'linear': 1 - f, 'ones', 'zeros'; f from 0 to 1 over the decay)."""
    weights = torch.zeros(n_action_steps)
    if prefix_len <= 0:
        return weights
    weights[:min(prefix_len, n_action_steps)] = 1.0
    if decay_end > prefix_len:
        decay_len = decay_end - prefix_len
        for i in range(decay_len):
            pos = prefix_len + i
            if pos >= n_action_steps:
                break
            frac = i / max(decay_len - 1, 1)
            if schedule == 'exp':
                weights[pos] = math.exp(-3.0 * frac)
            elif schedule == 'linear':
                weights[pos] = 1.0 - frac
            elif schedule == 'ones':
                weights[pos] = 1.0
            elif schedule == 'zeros':
                weights[pos] = 0.0
            else:
                raise ValueError(f'Unknown schedule: {schedule}')
    return weights


def compute_guidance_weight(t, max_guidance_weight):
    """compute_guidance_weight (rtc_guidance.py:83-104), t in [0, 1] with
    0 = noise: min((1-t)/t * (t^2 + (1-t)^2) / (1-t)^2, max), in double."""
    eps = 1e-6
    t_clamped = max(t, eps)
    one_minus_t = max(1.0 - t, eps)
    inv_r2 = (t_clamped**2 + one_minus_t**2) / (one_minus_t**2)
    c = one_minus_t / t_clamped
    return min(c * inv_r2, max_guidance_weight)


def apply_rtc_guidance(x_t, denoise_fn, prev_actions, prefix_weights, t,
                       max_guidance_weight, use_vjp=False):
    """apply_rtc_guidance (rtc_guidance.py:107-155): v + gw * c with the
    error e = w * (prev - x_1) on the first L_prev positions (zero after),
    x_1 = x_t + v (1 - t).  Without VJP c = e; with use_vjp c is e pulled
    back through x_1's Jacobian, (d x_1 / d x_t)^T e = e + (1 - t) J_v^T e,
    by torch autograd through the denoiser (:142-150)."""
    eps = 1e-6
    one_minus_t = max(1.0 - t, eps)
    w = prefix_weights[None, :, None]
    gw = compute_guidance_weight(t, max_guidance_weight)

    def full_error(x_1):
        L_prev = prev_actions.shape[1]
        error_full = torch.zeros_like(x_1)
        if L_prev:
            error_full[:, :L_prev] = ((prev_actions - x_1[:, :L_prev])
                                      * w[:, :L_prev])
        return error_full

    if use_vjp:
        with torch.enable_grad():
            x_g = x_t.detach().requires_grad_(True)
            v_t = denoise_fn(x_g)
            x_1 = x_g + v_t * one_minus_t
            (corr,) = torch.autograd.grad(x_1, x_g,
                                          grad_outputs=full_error(x_1))
        return v_t.detach() + gw * corr.detach()
    v_t = denoise_fn(x_t)
    return v_t + gw * full_error(x_t + v_t * one_minus_t)


def euler_guidance_rtc(x_t, denoise, bsize, dt, prev_actions, prefix_len,
                       rtc_config, n_action_steps):
    """_predict_action_guidance_rtc (pi0_flowmatching.py:671-700), with or
    without use_vjp: the guidance works in the 0 = noise time convention,
    so the model velocity enters negated."""
    prefix_weights = compute_prefix_weights(
        n_action_steps, prefix_len, rtc_config.get('decay_end', prefix_len * 2),
        rtc_config.get('schedule', 'exp'))
    max_gw = rtc_config.get('max_guidance_weight', 5.0)
    use_vjp = rtc_config.get('use_vjp', False)
    time = torch.tensor(1.0, dtype=torch.float32)
    while time >= -dt / 2:
        t_batch = time.expand(bsize)
        v_fm = apply_rtc_guidance(x_t, lambda x: -denoise(x, t_batch),
                                  prev_actions, prefix_weights,
                                  1.0 - time.item(), max_gw, use_vjp=use_vjp)
        x_t += dt * (-v_fm)
        time += dt
    return x_t


def rtc_inputs(cfg, prev_actions, prefix_len, rtc_config):
    """predict_action's RTC selection (pi0_flowmatching.py:747-756): prev
    padded to max_action_dim when ori_action_dim is set; the method is
    rtc_config['method'] (default 'prefix') when prev_actions, prefix_len > 0
    and rtc_config are all given, else None (plain loop)."""
    if (prev_actions is not None and cfg.ori_action_dim is not None
            and prev_actions.shape[-1] < cfg.max_action_dim):
        prev_actions = F.pad(prev_actions,
                             (0, cfg.max_action_dim - prev_actions.shape[-1]),
                             value=0.0)
    method = None
    if prev_actions is not None and prefix_len > 0 and rtc_config:
        method = rtc_config.get('method', 'prefix')
    return prev_actions, method


@torch.no_grad()
def predict_action(P, cfg, images, lang_tokens, states, img_masks=None,
                   lang_masks=None, noise=None, num_steps=None,
                   prev_actions=None, prefix_len=0, rtc_config=None):
    """PI0FlowMatching.predict_action (pi0_flowmatching.py:702-785): prefix
    cache, then the plain, prefix-RTC or guidance-RTC Euler loop, all on the
    CPU in fp32."""
    B = images.shape[0]
    if img_masks is None:
        img_masks = torch.ones(B, images.shape[1] // 3, dtype=torch.bool)
    if lang_masks is None:
        lang_masks = torch.ones(lang_tokens.shape, dtype=torch.bool)
    kvs, prefix_pad = prefix_forward(P, cfg, images, lang_tokens, img_masks,
                                     lang_masks)
    steps = cfg.num_steps if num_steps is None else num_steps
    dt = torch.tensor(-1.0 / steps, dtype=torch.float32)
    if prev_actions is not None:
        prev_actions = prev_actions.float()
    prev_actions, method = rtc_inputs(cfg, prev_actions, prefix_len,
                                      rtc_config)
    x_t = noise.float().clone()

    def denoise(x, t):
        return denoise_step(P, cfg, states.float(), prefix_pad, kvs, x, t)

    if method == 'prefix':
        return euler_prefix_rtc(x_t, denoise, B, dt, prev_actions, prefix_len,
                                cfg.n_action_steps)
    if method == 'guidance':
        return euler_guidance_rtc(x_t, denoise, B, dt, prev_actions,
                                  prefix_len, rtc_config, cfg.n_action_steps)
    return euler_plain(x_t, denoise, B, dt)
