"""PI0 / PI0.5 action-chunk inference on MI355X.

Host-side mirror of the reference's fused inference model
(fluxvla/models/vlas/pi05_flowmatching_inference.py:329-656): weight
preparation hooks, static buffers, one pipeline function per stage
(vision_encoder / transformer_encoder / transformer_decoder, :22-312) and
one HIP graph per batch size that replays the whole chunk (:469-512).  Unlike
the reference fast path it covers PI0 (state token, block-causal suffix) as
well as PI0.5 (adaRMS), batches > 1, and follows the reference's PyTorch
path where the Triton path departs from it (suffix RoPE positions start at
sum(prefix_pad) as in pi0_flowmatching.py:817-819; SigLIP LayerNorm eps is
the config's 1e-6).

Every op runs as a HIP kernel from libfluxvla_amd.so; torch is used for
buffers, the stream and graph capture, and to stage the request's inputs.
"""
import math

import torch

from . import kernels as K
from . import rtc as R
from ._lib import ACT_GELU_TANH, ACT_SILU
from .config import PI0Config

BF16 = torch.bfloat16
INT32_MAX = 2**31 - 1
VIS = 'vision_backbone.vision.vision_model'


# ---------------------------------------------------------------------------
# Weight preparation hooks
# ---------------------------------------------------------------------------
def interleave_rows(head_dim):
    """Row order that places rotate-half pair (i, i + d/2) at (2i, 2i + 1),
    the same layout condition_gemma_inference.py:46-63 produces, so RoPE is a
    rotation of adjacent columns inside the GEMM epilogue.  Applied to both Q
    and K it leaves Q K^T unchanged."""
    return torch.arange(head_dim).view(2, head_dim // 2).t().reshape(-1)


def prepare_siglip(sd, cfg: PI0Config, device):
    """SigLIPViTBackboneInference.prepare_triton counterpart
    (fluxvla/models/visions/siglip_vit_inference.py:10-101): conv weight
    flattened in (c, ky, kx) order and zero-padded to a multiple of 8
    columns; Q|K|V stacked with their biases; weights stay [out, in]."""
    vh, kp = cfg.vit_hidden, cfg.patch_k_pad
    pw = torch.zeros(vh, kp, dtype=BF16)
    pw[:, :cfg.patch_k] = sd[f'{VIS}.embeddings.patch_embedding.weight'].reshape(vh, -1)
    w = {
        'patch_w': pw,
        'patch_b': sd[f'{VIS}.embeddings.patch_embedding.bias'],
        'pos_emb': sd[f'{VIS}.embeddings.position_embedding.weight'],
        'post_ln_w': sd[f'{VIS}.post_layernorm.weight'],
        'post_ln_b': sd[f'{VIS}.post_layernorm.bias'],
    }
    layers = []
    for i in range(cfg.vit_layers):
        pre = f'{VIS}.encoder.layers.{i}'
        a = f'{pre}.self_attn'
        layers.append({
            'ln1_w': sd[f'{pre}.layer_norm1.weight'],
            'ln1_b': sd[f'{pre}.layer_norm1.bias'],
            'qkv_w': torch.cat([sd[f'{a}.q_proj.weight'], sd[f'{a}.k_proj.weight'],
                                sd[f'{a}.v_proj.weight']], 0),
            'qkv_b': torch.cat([sd[f'{a}.q_proj.bias'], sd[f'{a}.k_proj.bias'],
                                sd[f'{a}.v_proj.bias']], 0),
            'o_w': sd[f'{a}.out_proj.weight'],
            'o_b': sd[f'{a}.out_proj.bias'],
            'ln2_w': sd[f'{pre}.layer_norm2.weight'],
            'ln2_b': sd[f'{pre}.layer_norm2.bias'],
            'fc1_w': sd[f'{pre}.mlp.fc1.weight'],
            'fc1_b': sd[f'{pre}.mlp.fc1.bias'],
            'fc2_w': sd[f'{pre}.mlp.fc2.weight'],
            'fc2_b': sd[f'{pre}.mlp.fc2.bias'],
        })
    w['layers'] = layers
    return _to(w, device)


def prepare_gemma(sd, cfg: PI0Config, role, device):
    """ConditionGemmaInferenceModel.prepare_triton counterpart
    (condition_gemma_inference.py:65-170).  For plain-RMSNorm layers the
    Gemma (1 + w) scale is folded into the following Q/K/V (input norm) and
    gate/up (post-attention norm) weights in fp32 before the single bf16
    rounding (:85-101); the expert's final norm is folded into
    action_out_proj.  Q/K rows go to pair-interleaved order.  adaRMS layers
    (PI0.5 expert) keep their dense modulation weights instead."""
    prefix = 'llm_backbone' if role == 'llm' else 'llm_expert'
    n = cfg.llm_layers if role == 'llm' else cfg.exp_layers
    adarms = role == 'expert' and cfg.pi05
    H, D = cfg.heads, cfg.head_dim
    perm = interleave_rows(D)
    layers = []
    for i in range(n):
        pre = f'{prefix}.layers.{i}'
        wq = sd[f'{pre}.self_attn.q_proj.weight'].float()
        wk = sd[f'{pre}.self_attn.k_proj.weight'].float()
        wv = sd[f'{pre}.self_attn.v_proj.weight'].float()
        wg = sd[f'{pre}.mlp.gate_proj.weight'].float()
        wu = sd[f'{pre}.mlp.up_proj.weight'].float()
        L = {}
        if adarms:
            for nm, key in (('attn', 'input_layernorm'),
                            ('ffn', 'post_attention_layernorm')):
                L[f'{nm}_mod_w'] = sd[f'{pre}.{key}.dense.weight']
                L[f'{nm}_mod_b'] = sd[f'{pre}.{key}.dense.bias']
        else:
            s_in = 1.0 + sd[f'{pre}.input_layernorm.weight'].float()
            s_post = 1.0 + sd[f'{pre}.post_attention_layernorm.weight'].float()
            wq, wk, wv = wq * s_in, wk * s_in, wv * s_in
            wg, wu = wg * s_post, wu * s_post
        wq = wq.view(H, D, -1)[:, perm].reshape(H * D, -1)
        wk = wk[perm]
        L['qkv_w'] = torch.cat([wq, wk, wv], 0).to(BF16)
        L['o_w'] = sd[f'{pre}.self_attn.o_proj.weight']
        L['gate_w'] = wg.to(BF16)
        L['up_w'] = wu.to(BF16)
        L['down_w'] = sd[f'{pre}.mlp.down_proj.weight']
        layers.append(L)
    w = {'layers': layers}
    if role == 'llm':
        w['embed'] = sd['llm_backbone.embed_tokens.weight']
    elif adarms:
        w['final_mod_w'] = sd['llm_expert.norm.dense.weight']
        w['final_mod_b'] = sd['llm_expert.norm.dense.bias']
    else:
        w['final_scale'] = 1.0 + sd['llm_expert.norm.weight'].float()
    return _to(w, device)


LINEARS = ('qkv_w', 'o_w', 'gate_w', 'up_w', 'down_w')


WEIGHT_DTYPES = ('bf16', 'fp8', 'fp8_w8a8')


def quantize_linears(w, act='bf16'):
    """fp8 variant (PI0.5 config 5): every linear layer of a Gemma tower
    (Q|K|V, O, gate, up, down) as OCP e4m3fn with one fp32 scale per output
    channel, s = max|W[j]| / 448, taken after the (1 + w) fold and the Q/K
    interleave, so the quantized weight is exactly the one the GEMM applies.
    The reference has no fp8 path.  ``act='bf16'`` (W8A16, config 5 as
    stated: bf16 activations, fp32 accumulate): the kernels convert the
    e4m3 bytes to bf16 in registers; ``act='e4m3'`` (W8A8, opt-in): they
    quantize the activations per row and k step on the fly."""
    for L in w['layers']:
        for nm in LINEARS:
            L[nm] = K.Fp8Weight.quantize(L[nm], act=act)
    return w


def prepare_projector(sd, prefix, device):
    """LinearProjectorInference.prepare_triton counterpart
    (linear_projector_inference.py:8-14): weight [out, in] and bias."""
    return _to({'w': sd[f'{prefix}.projector.weight'],
                'b': sd[f'{prefix}.projector.bias']}, device)


def _to(obj, device):
    if isinstance(obj, dict):
        return {k: _to(v, device) for k, v in obj.items()}
    if isinstance(obj, list):
        return [_to(v, device) for v in obj]
    if isinstance(obj, torch.Tensor):
        return obj.to(device).contiguous()
    return obj


def euler_times(num_steps):
    """fp32 time values of the reference Euler loop
    (pi0_flowmatching.py:642-649): t = 1, t += dt while t >= -dt/2."""
    dt = torch.tensor(-1.0 / num_steps, dtype=torch.float32)
    t = torch.tensor(1.0, dtype=torch.float32)
    out = []
    while t >= -dt / 2:
        out.append(float(t))
        t = t + dt
    return out, float(dt)


def sinusoid(times, dim, min_period=4e-3, max_period=4.0):
    """create_sinusoidal_pos_embedding (model_utils.py:40-68), fp32, for the
    input-independent per-step time embeddings."""
    fraction = torch.linspace(0.0, 1.0, dim // 2, dtype=torch.float32)
    period = min_period * (max_period / min_period)**fraction
    x = torch.tensor(times, dtype=torch.float32)[:, None] * (
        1.0 / period * 2 * math.pi)
    return torch.cat([torch.sin(x), torch.cos(x)], dim=-1)


def suffix_att_pattern(cfg: PI0Config):
    """Suffix attention-mask pattern: PI0 [1, 1, 0 x 49] (state block, then
    the action block; pi0_flowmatching.py:274-313), PI0.5 [1, 0 x 49]
    (pi05_flowmatching.py:112-120)."""
    na = cfg.n_action_steps
    return [1] + [0] * (na - 1) if cfg.pi05 else [1, 1] + [0] * (na - 1)


def attention_groups(prefix_pad, suffix_att):
    """The prefix/suffix masks as the kernels consume them.

    make_att_2d_masks (model_utils.py:77-95) over [prefix (att all 0) |
    suffix] lets query token i see key j iff cumsum(att)[j] <= cumsum(att)[i]
    and both are valid; denoise_step shows every suffix row all valid prefix
    keys (pi0_flowmatching.py:802-813).  So with
        kgrp[j] = cumsum(att)[j] if key j is valid else INT32_MAX
        qgrp[i] = cumsum(att)[i]
    key j is visible to valid query i iff kgrp[j] <= qgrp[i].  Positions
    follow the PyTorch path: prefix cumsum(pad) - 1, suffix sum(prefix_pad)
    + cumsum(suffix_pad) - 1 (pi0_flowmatching.py:729-730, 817-819).

    prefix_pad: bool [B, S]; suffix_att: int/bool [Ss] (all suffix tokens
    valid).  Returns int32 kgrp [B, S + Ss], qgrp_prefix [B, S],
    qgrp_suffix [B, Ss], pos_prefix [B, S], pos_suffix [B, Ss]."""
    B, S = prefix_pad.shape
    dev = prefix_pad.device
    pad = prefix_pad.bool()
    scum = torch.cumsum(torch.as_tensor(suffix_att, dtype=torch.int32,
                                        device=dev), 0).to(torch.int32)
    Ss = scum.numel()
    kg_pre = torch.where(pad, 0, INT32_MAX).to(torch.int32)
    kgrp = torch.cat([kg_pre, scum[None].expand(B, Ss)], dim=1)
    qgrp_pre = torch.zeros(B, S, dtype=torch.int32, device=dev)
    qgrp_suf = scum[None].expand(B, Ss).contiguous()
    pos_pre = (torch.cumsum(pad.int(), 1) - 1).to(torch.int32)
    off = pad.int().sum(1, keepdim=True)
    pos_suf = (off + torch.arange(Ss, device=dev, dtype=torch.int32)).to(
        torch.int32)
    return kgrp, qgrp_pre, qgrp_suf, pos_pre, pos_suf


def prefix_pad_mask(img_masks, lang_masks, num_patches):
    """embed_prefix pad mask (pi0_flowmatching.py:216-247): each camera's
    mask repeated over its patches, then the prompt mask."""
    return torch.cat([img_masks.bool().repeat_interleave(num_patches, dim=1),
                      lang_masks.bool()], dim=1)


# ---------------------------------------------------------------------------
# The inference model
# ---------------------------------------------------------------------------
class PI0Inference:
    """Static-buffer, graph-replayed PI0 / PI0.5 action-chunk inference.

    ``predict_action`` keeps the reference signature
    (pi0_flowmatching.py:702-715) and returns the denoised chunk
    [B, n_action_steps, max_action_dim] in fp32.
    """

    def __init__(self, cfg: PI0Config, state_dict, device='cuda',
                 max_batch=1, use_graph=True, weight_dtype='bf16',
                 fp8_cache=None):
        """``weight_dtype``: 'bf16'; 'fp8' (e4m3 Gemma linears, bf16
        activations: W8A16); 'fp8_w8a8' (e4m3 linears and e4m3 activations,
        quantized per row and k step in the GEMMs).  ``fp8_cache``: path of
        a safetensors file holding the quantized linears; read when it was
        written for these weights (checkpoint.load_fp8_cache), else the
        weights are quantized and the file (re)written."""
        if weight_dtype not in WEIGHT_DTYPES:
            raise ValueError(f'weight_dtype must be one of {WEIGHT_DTYPES}, '
                             f'got {weight_dtype!r}')
        self.cfg = cfg
        self.device = torch.device(device)
        self.use_graph = use_graph
        self.max_batch = max_batch
        # bs=1 expert: the attention's idle workgroups prefetch the next
        # GEMMs' weights, each 16-column tile into the L2 of the XCD that
        # will read it (prefetch_place) or the memory-side cache
        self.prefetch = True
        self.prefetch_place = True
        self.prefetch_kv = True
        # PI0.5 at bs=1: the adaptive RMSNorms run inside the next GEMM
        # (A scaled by 1 + scale as it is loaded, the shift as a bias, the
        # gate read from the style row by the residual epilogues)
        self.fold_adarms = True
        # SigLIP: with fold_layernorm the LayerNorms run inside the GEMMs
        # after them (Q|K|V, fc1, the projector), on row sums taken in their
        # K loops.  Off by default: ~0.1 ms faster per chunk, but the gain
        # folded into the bf16 weights moves every token's product the same
        # way, and the full-depth chunk lands 10-35 % further from the fp32
        # oracle (up to 2.0e-2 on the 2e-2 bar)
        self.fold_layernorm = False
        # predict_action ends with the attention merge status check (it
        # waits for the chunk); off, callers run kernels.attention_check
        self.check_merge = True
        self.weight_dtype = weight_dtype
        self.fp8_cache = fp8_cache
        self.fp8_cache_hit = False
        K.workspace(self.device)
        K.workspace(self.device, 'attn')
        self._sd = state_dict
        self.prepare_triton_inference(state_dict)
        self._graphs = {}
        self._bufs = {}

    # -- weight prep (prepare_triton_inference, :596-656) --------------------
    @torch.no_grad()
    def prepare_triton_inference(self, sd):
        cfg, dev = self.cfg, self.device
        self._vjp = None  # rebuilt from these weights on first use
        self.vis = prepare_siglip(sd, cfg, dev)
        self.llm = prepare_gemma(sd, cfg, 'llm', dev)
        self.exp = prepare_gemma(sd, cfg, 'expert', dev)
        if self.fp8:
            from .checkpoint import build_fp8_cache, load_fp8_cache
            act = 'e4m3' if self.weight_dtype == 'fp8_w8a8' else 'bf16'
            cached = (load_fp8_cache(self.fp8_cache, sd, cfg, act, dev)
                      if self.fp8_cache else None)
            if cached is not None:
                for W, layers in ((self.llm, cached['llm']),
                                  (self.exp, cached['expert'])):
                    for L, C in zip(W['layers'], layers):
                        L.update(C)
                self.fp8_cache_hit = True
            else:
                quantize_linears(self.llm, act)
                quantize_linears(self.exp, act)
                if self.fp8_cache:
                    build_fp8_cache(self, sd, self.fp8_cache)
        self.proj = prepare_projector(sd, 'projector', dev)
        self.act_in = prepare_projector(sd, 'action_in_proj', dev)
        out = prepare_projector(sd, 'action_out_proj', dev)
        if not cfg.pi05:
            # final expert RMSNorm (1 + w) folded into action_out_proj
            out['w'] = (out['w'].float() *
                        self.exp.pop('final_scale')[None]).to(BF16)
        self.act_out = out
        self.times, self.dt = euler_times(cfg.num_steps)
        self._rtc_omt = R.guidance_omt(self.times)
        # the last row is time 0: the positions real-time chunking locks
        temb = sinusoid(self.times + [0.0], cfg.proj_width).to(BF16).to(dev)
        w = cfg.proj_width
        if cfg.pi05:
            tin = prepare_projector(sd, 'time_mlp_in', dev)
            tout = prepare_projector(sd, 'time_mlp_out', dev)
            h = K.gemm(temb, tin['w'], bias=tin['b'], act=ACT_SILU)
            cond = K.gemm(h, tout['w'], bias=tout['b'], act=ACT_SILU)
            # adaRMS style rows depend only on (step, layer): precomputed once
            styles = []
            for L in self.exp['layers']:
                styles.append(K.gemm(cond, L['attn_mod_w'],
                                     bias=L['attn_mod_b']))
                styles.append(K.gemm(cond, L['ffn_mod_w'],
                                     bias=L['ffn_mod_b']))
            styles.append(K.gemm(cond, self.exp['final_mod_w'],
                                 bias=self.exp['final_mod_b']))
            # [steps, 2 * layers + 1, 3 * width], and the time-0 rows
            styles = torch.stack(styles, 1)
            self.styles = styles[:-1].contiguous()
            self.styles0 = styles[-1].contiguous()
        else:
            self.state = prepare_projector(sd, 'state_proj', dev)
            mi = prepare_projector(sd, 'action_time_mlp_in', dev)
            mo = prepare_projector(sd, 'action_time_mlp_out', dev)
            # cat([action_emb, time_emb]) @ W^T = action_emb @ Wa^T +
            # time_emb @ Wt^T: the time half is a per-step fp32 bias.
            wt = mi['w'][:, w:].contiguous()
            bias = K.gemm(temb, wt, bias=mi['b'], out_f32=True)
            # action_in_proj folded in: (x Wi^T + bi) Wa^T = x (Wa Wi)^T +
            # Wa bi, one K = max_action_dim GEMM per step instead of two
            wa = mi['w'][:, :w].float()
            self.mlp_in_x = (wa @ self.act_in['w'].float()).to(BF16)
            fold_b = wa @ self.act_in['b'].float()
            self.step_bias = (bias[:-1] + fold_b).contiguous()
            self.step_bias0 = (bias[-1] + fold_b).contiguous()
            self.mlp_out = mo
        self.rope = K.rope_table(cfg.prefix_len + cfg.suffix_len + 8,
                                 cfg.head_dim, cfg.rope_theta, device=dev)
        self._prepare_frag_weights()
        self._prepare_adarms_fold()
        self._prepare_layernorm_fold()
        torch.cuda.synchronize(dev)

    def _prepare_layernorm_fold(self):
        """SigLIP's LayerNorms folded into the GEMMs after them: with g / beta
        the norm's gain / shift, LN(x) @ W^T + b = rstd * (x @ (W g)^T -
        mean * csum) + (b + W beta), csum[n] = sum_k (W g)[n, k] taken from
        the bf16 weights the MFMAs multiply (fvx_gemm_desc.ln_csum); mean
        and rstd come from row sums of x the GEMM takes in its K loop."""
        def fold(w, bias, g, beta):
            wg = (w.float() * g.float()[None]).to(BF16)
            return {'w': wg, 'csum': wg.float().sum(1).contiguous(),
                    'b': (bias.float() + w.float() @ beta.float()).contiguous()}
        V = self.vis
        self.vis_ln = [{'qkv': fold(L['qkv_w'], L['qkv_b'], L['ln1_w'], L['ln1_b']),
                        'fc1': fold(L['fc1_w'], L['fc1_b'], L['ln2_w'], L['ln2_b'])}
                       for L in V['layers']]
        self.proj_ln = fold(self.proj['w'], self.proj['b'], V['post_ln_w'],
                            V['post_ln_b'])

    def _prepare_adarms_fold(self):
        """Per (step, layer) fp32 biases shift @ W^T of the folded adaptive
        RMSNorms (PI0.5): the input norm's shift through Q|K|V, the
        post-attention norm's through gate and up, the final norm's through
        action_out_proj.  The (1 + scale) factor and the gate are read from
        the style rows themselves."""
        if not self.cfg.pi05 or self.weight_dtype == 'fp8_w8a8':
            self.fold = None
            return
        w = self.cfg.exp_hidden
        st = self.styles  # [steps, 2 * layers + 1, 3 * w]
        self.fold = []
        for i, L in enumerate(self.exp['layers']):
            ha, hf = st[:, 2 * i, w:2 * w], st[:, 2 * i + 1, w:2 * w]
            self.fold.append({
                'qkv': K.gemm(ha, L['qkv_w'], out_f32=True),
                'gate': K.gemm(hf, L['gate_w'], out_f32=True),
                'up': K.gemm(hf, L['up_w'], out_f32=True)})
        self.fold_out = K.gemm(st[:, -1, w:2 * w], self.act_out['w'],
                               out_f32=True)

    def _prepare_frag_weights(self):
        """Fragment-major copies of the action-expert weights for the M <= 64
        (bs=1) skinny GEMMs: every weight load becomes one coalesced 1 KiB
        block per wave.  The row-major originals stay for batched calls."""
        F = K.FragB.pack

        def frag(w):
            return w.pack_frag() if isinstance(w, K.Fp8Weight) else F(w)
        self.exp_f = []
        for L in self.exp['layers']:
            self.exp_f.append({nm: frag(L[nm]) for nm in LINEARS})
        self.act_out_f = F(self.act_out['w'])
        if self.cfg.pi05:
            self.act_in_f = F(self.act_in['w'])
        else:
            self.mlp_in_x_f = F(self.mlp_in_x)
            self.mlp_out_f = F(self.mlp_out['w'])

    # -- the reference's module attributes with their prepare_triton hooks
    #    (pi05_flowmatching_inference.py:596-619): each returns the
    #    reference-keyed dict of hooks.py for its part of the state dict
    @property
    def vision_backbone(self):
        from .hooks import SigLIPViTBackboneInference
        return SigLIPViTBackboneInference(self._sd, self.cfg, self.device)

    @property
    def llm_backbone(self):
        from .hooks import ConditionGemmaInferenceModel
        return ConditionGemmaInferenceModel(self._sd, self.cfg, 'llm_backbone',
                                            self.device)

    @property
    def llm_expert(self):
        from .hooks import ConditionGemmaInferenceModel
        return ConditionGemmaInferenceModel(self._sd, self.cfg, 'llm_expert',
                                            self.device)

    def projector_hook(self, module):
        """LinearProjectorInference of ``module`` ('projector',
        'action_in_proj', 'action_out_proj', 'time_mlp_in', ...)."""
        from .hooks import LinearProjectorInference
        return LinearProjectorInference.from_state_dict(self._sd, module,
                                                        self.device)

    @property
    def projector(self):
        return self.projector_hook('projector')

    @property
    def fp8(self):
        return self.weight_dtype in ('fp8', 'fp8_w8a8')

    def dequantized_state_dict(self, sd):
        """fp8 models: the state dict whose fp32 forward is the model the
        fp8 pipeline runs -- every quantized linear replaced by its
        dequantized weight (scale * e4m3 bytes, read back from the device),
        with the preparation's (1 + w) fold and Q/K interleave undone, so a
        reference implementation's own norms and RoPE apply to it unchanged.
        Tensors are fp32 on the CPU; the other entries are those of ``sd``."""
        if not self.fp8:
            raise ValueError('dequantized_state_dict needs an fp8 model')
        cfg = self.cfg
        H, D = cfg.heads, cfg.head_dim
        inv = torch.argsort(interleave_rows(D))
        out = dict(sd)
        for role, prefix, W in (('llm', 'llm_backbone', self.llm),
                                ('expert', 'llm_expert', self.exp)):
            adarms = role == 'expert' and cfg.pi05
            for i, L in enumerate(W['layers']):
                pre = f'{prefix}.layers.{i}'
                dq = {nm: L[nm].dequantize().cpu() for nm in LINEARS}
                qkv = dq['qkv_w']
                wq = qkv[:H * D].view(H, D, -1)[:, inv].reshape(H * D, -1)
                wk, wv = qkv[H * D:H * D + D][inv], qkv[H * D + D:]
                wg, wu = dq['gate_w'], dq['up_w']
                if not adarms:
                    s_in = 1.0 + sd[f'{pre}.input_layernorm.weight'].float().cpu()
                    s_post = 1.0 + sd[
                        f'{pre}.post_attention_layernorm.weight'].float().cpu()
                    wq, wk, wv = wq / s_in, wk / s_in, wv / s_in
                    wg, wu = wg / s_post, wu / s_post
                out[f'{pre}.self_attn.q_proj.weight'] = wq
                out[f'{pre}.self_attn.k_proj.weight'] = wk
                out[f'{pre}.self_attn.v_proj.weight'] = wv
                out[f'{pre}.self_attn.o_proj.weight'] = dq['o_w']
                out[f'{pre}.mlp.gate_proj.weight'] = wg
                out[f'{pre}.mlp.up_proj.weight'] = wu
                out[f'{pre}.mlp.down_proj.weight'] = dq['down_w']
        return out

    @property
    def kv_len(self):
        """Token capacity of the K/V caches: prefix + suffix, rounded up to a
        multiple of 8 (16-byte rows of the transposed value cache)."""
        n = self.cfg.prefix_len + self.cfg.suffix_len
        return (n + 7) // 8 * 8

    # -- static buffers (_init_buffers, :356-442) ----------------------------
    def _buffers(self, B):
        if B in self._bufs:
            return self._bufs[B]
        cfg, dev = self.cfg, self.device
        S, Ss, D = cfg.prefix_len, cfg.suffix_len, cfg.head_dim
        T = self.kv_len
        nimg = B * cfg.n_views
        nv_tok = nimg * cfg.num_patches
        e = lambda *s, dt=BF16: torch.zeros(*s, dtype=dt, device=dev)  # noqa
        b = {
            'images': e(B, 3 * cfg.n_views, cfg.image_size, cfg.image_size,
                        dt=torch.float32),
            'ids': e(B, cfg.max_prompt_len, dt=torch.int64),
            'patches': e(nv_tok, cfg.patch_k_pad),
            'vis_x': e(nv_tok, cfg.vit_hidden),
            'vis_xn': e(nv_tok, cfg.vit_hidden),
            'vis_qkv': e(nv_tok, 3 * cfg.vit_hidden),
            'vis_ctx': e(nv_tok, cfg.vit_hidden),
            'vis_h': e(nv_tok, cfg.vit_mlp),
            'pre_x': e(B, S, cfg.llm_hidden),
            'pre_q': e(B, S, cfg.heads * D),
            'pre_ctx': e(B, S, cfg.heads * D),
            'pre_h': e(B * S, cfg.llm_mlp),
            # row sums of squares of x handed between prefix GEMMs
            'pre_ss': e(2, K.ss_parts(cfg.llm_hidden), B * S, dt=torch.float32),
            # e4m3 copies of x and of the gate/up output (W8A8 weights)
            'pre_a8x': (K.Fp8Act.empty(B * S, cfg.llm_hidden, dev)
                        if self.weight_dtype == 'fp8_w8a8' else None),
            'pre_a8h': (K.Fp8Act.empty(B * S, cfg.llm_mlp, dev)
                        if self.weight_dtype == 'fp8_w8a8' else None),
            # K cache [layer][batch][token][dim] (pair-interleaved dims);
            # V cache transposed [layer][batch][dim][token]
            'kc': e(cfg.exp_layers, B, T, D),
            'vc': e(cfg.exp_layers, B, D, T),
            'pos_pre': e(B * S, dt=torch.int32),
            'pos_suf': e(B * Ss, dt=torch.int32),
            'kgrp': e(B, S + Ss, dt=torch.int32),
            'qgrp_pre': e(B, S, dt=torch.int32),
            'qgrp_suf': e(B, Ss, dt=torch.int32),
            'ex_x': e(B, Ss, cfg.exp_hidden),
            'ex_xn': e(B, Ss, cfg.exp_hidden),
            'ex_gate': e(B, Ss, cfg.exp_hidden),
            'ex_q': e(B, Ss, cfg.heads * D),
            'ex_ctx': e(B, Ss, cfg.heads * D),
            'ex_h': e(B * Ss, cfg.exp_mlp),
            # fragment-major copies of x, the attention output and the GeGLU
            # output for the bs=1 skinny GEMMs (M = suffix_len <= 64)
            'ex_xf': K.FragA.empty(cfg.exp_hidden, dev),
            'ex_ctxf': K.FragA.empty(cfg.heads * D, dev),
            'ex_hf': K.FragA.empty(cfg.exp_mlp, dev),
            'states': e(B, cfg.state_dim),
            'xt': e(B, cfg.n_action_steps, cfg.max_action_dim,
                    dt=torch.float32),
            'xt_bf16': e(B, cfg.n_action_steps, cfg.max_action_dim),
            # real-time chunking: locked prefix length, the previous chunk
            # (zero rows past its length) and the guidance weights per step
            'rtc_lock': e(1, dt=torch.int32),
            'rtc_prev': e(B, cfg.n_action_steps, cfg.max_action_dim,
                          dt=torch.float32),
            'rtc_cw': e(len(self.times), cfg.n_action_steps,
                        dt=torch.float32),
            # guidance with use_vjp: the prefix weights (zero past the
            # previous chunk) and each step's guidance weight
            'rtc_w': e(cfg.n_action_steps, dt=torch.float32),
            'rtc_gw': e(len(self.times), dt=torch.float32),
        }
        if not cfg.pi05:
            # PI0 suffix stream = [state_emb, mlp_out(silu(mlp_in(...)))]:
            # the hidden rows of the action-time MLP sit at the suffix rows
            # (the state row of each sample stays zero), and the mlp_out
            # GEMM adds a constant residual that holds the state embedding
            # in the state row and mlp_out's bias in the action rows
            b['suf_h'] = e(B * Ss, cfg.proj_width)
            b['suf_res'] = (self.mlp_out['b'][None]
                            .expand(B * Ss, cfg.exp_hidden).contiguous())
        self._bufs[B] = b
        return b

    # -- pipeline ------------------------------------------------------------
    def vision_encoder(self, b, B):
        """SigLIP per view + projector into the prefix rows
        (pi05_flowmatching_inference.py:22-66, 69-84)."""
        cfg, V = self.cfg, self.vis
        nimg = B * cfg.n_views
        imgs = b['images'].view(nimg, 3, cfg.image_size, cfg.image_size)
        K.im2col_patches(imgs, cfg.patch, cfg.patch_k_pad, out=b['patches'])
        x, xn = b['vis_x'], b['vis_xn']
        n_img_tok = cfg.n_views * cfg.num_patches
        pre = b['pre_x'].view(-1, cfg.llm_hidden)
        if self.fold_layernorm:
            # every LayerNorm inside the next GEMM, on row sums of x taken in
            # that GEMM's K loop
            ln = lambda f: {'rownorm_eps': cfg.vit_eps, 'ln_csum': f['csum'],  # noqa
                            'bias_f32': f['b']}
            K.gemm(b['patches'], V['patch_w'], out=x, bias=V['patch_b'],
                   pos=V['pos_emb'], pos_period=cfg.num_patches)
            for L, F in zip(V['layers'], self.vis_ln):
                K.gemm(x, F['qkv']['w'], out=b['vis_qkv'], **ln(F['qkv']))
                K.mha_packed_qkv(b['vis_qkv'], b['vis_ctx'], nimg,
                                 cfg.num_patches, cfg.vit_heads, cfg.vit_head_dim)
                K.gemm(b['vis_ctx'], L['o_w'], out=x, bias=L['o_b'], residual=x)
                K.gemm(x, F['fc1']['w'], out=b['vis_h'], act=ACT_GELU_TANH,
                       **ln(F['fc1']))
                K.gemm(b['vis_h'], L['fc2_w'], out=x, bias=L['fc2_b'], residual=x)
            K.gemm(x, self.proj_ln['w'], out=pre, row_group=n_img_tok,
                   row_group_stride=cfg.prefix_len, **ln(self.proj_ln))
            return
        K.gemm(b['patches'], V['patch_w'], out=x, bias=V['patch_b'],
               pos=V['pos_emb'], pos_period=cfg.num_patches)
        for L in V['layers']:
            K.layer_norm(x, L['ln1_w'], L['ln1_b'], cfg.vit_eps, out=xn)
            K.gemm(xn, L['qkv_w'], out=b['vis_qkv'], bias=L['qkv_b'])
            K.mha_packed_qkv(b['vis_qkv'], b['vis_ctx'], nimg,
                             cfg.num_patches, cfg.vit_heads, cfg.vit_head_dim)
            K.gemm(b['vis_ctx'], L['o_w'], out=x, bias=L['o_b'], residual=x)
            K.layer_norm(x, L['ln2_w'], L['ln2_b'], cfg.vit_eps, out=xn)
            K.gemm(xn, L['fc1_w'], out=b['vis_h'], bias=L['fc1_b'],
                   act=ACT_GELU_TANH)
            K.gemm(b['vis_h'], L['fc2_w'], out=x, bias=L['fc2_b'], residual=x)
        K.layer_norm(x, V['post_ln_w'], V['post_ln_b'], cfg.vit_eps, out=xn)
        K.gemm(xn, self.proj['w'], out=pre, bias=self.proj['b'], row_group=n_img_tok,
               row_group_stride=cfg.prefix_len)

    def transformer_encoder(self, b, B):
        """Gemma-2B prefix: fills the K/V cache rows [0, S) of every layer
        (pi05_flowmatching_inference.py:69-152).  The last layer stops after
        its K/V: its outputs feed nothing."""
        cfg, W = self.cfg, self.llm
        S, D, hid = cfg.prefix_len, cfg.head_dim, cfg.llm_hidden
        T = self.kv_len
        n_img_tok = cfg.n_views * cfg.num_patches
        x = b['pre_x'].view(B * S, hid)
        K.embed_tokens(W['embed'], b['ids'],
                       b['pre_x'].view(-1, hid)[n_img_tok:],
                       scale=math.sqrt(hid), row_group=cfg.max_prompt_len,
                       row_group_stride=S)
        n = len(W['layers'])
        # row sums of squares of x handed from the residual GEMMs to the
        # next fused RMSNorm (O proj -> gate/up, down -> next QKV)
        ss = b['pre_ss'] if B * S > 64 else [None, None]
        # W8A8 weights: the residual GEMMs and gate/up also hand their
        # outputs over as e4m3 copies, which the fp8 wide GEMMs read instead
        # of quantizing their A (same values)
        a8x = a8h = None
        if self.weight_dtype == 'fp8_w8a8' and B * S > 64:
            a8x, a8h = b['pre_a8x'], b['pre_a8h']
        for i, L in enumerate(W['layers']):
            kc, vc = b['kc'][i], b['vc'][i]
            last = i == n - 1
            wqkv = L['qkv_w']
            if last:
                wqkv = (wqkv.rows(cfg.heads * D) if isinstance(wqkv, K.Fp8Weight)
                        else wqkv[cfg.heads * D:])
            K.gemm_qkv_rope(x, wqkv, self.rope, b['pos_pre'],
                            b['pre_q'].view(B * S, -1),
                            kc.view(B * T, D), vc, 0 if last else cfg.heads,
                            D, rownorm_eps=cfg.rms_eps, row_group=S,
                            row_group_stride=T, v_ld=T,
                            ss_in=ss[1] if i > 0 else None,
                            a8=a8x if i > 0 else None)
            if last:
                break
            K.mqa_attention(b['pre_q'], kc[:, :S], vc, b['pre_ctx'],
                            kgrp=b['kgrp'][:, :S], qgrp=b['qgrp_pre'],
                            v_transposed=True)
            K.gemm(b['pre_ctx'].view(B * S, -1), L['o_w'], out=x, residual=x,
                   ss_out=ss[0], a8_out=a8x)
            K.gemm_geglu(x, L['gate_w'], L['up_w'], out=b['pre_h'],
                         rownorm_eps=cfg.rms_eps, ss_in=ss[0], a8=a8x, a8_out=a8h)
            K.gemm(b['pre_h'], L['down_w'], out=x, residual=x, ss_out=ss[1],
                   a8=a8h, a8_out=a8x)

    def _frag_ok(self, B):
        """bs=1 expert GEMMs (M = suffix_len <= 64) run fragment-major."""
        return B * self.cfg.suffix_len <= 64

    def _expert_layer_pi0_frag(self, b, i, L):
        """_expert_layer_pi0 at bs=1 with fragment-major operands: x, the
        attention output and the GeGLU output are kept in the layout of the
        skinny GEMM's A fragments (the epilogues write it next to the
        row-major x)."""
        cfg = self.cfg
        S, Ss, D, hid = cfg.prefix_len, cfg.suffix_len, cfg.head_dim, cfg.exp_hidden
        T = self.kv_len
        Lf = self.exp_f[i]
        x = b['ex_x'].view(Ss, hid)
        xf = b['ex_xf'].rows(Ss)
        ctxf, hf = b['ex_ctxf'].rows(Ss), b['ex_hf'].rows(Ss)
        kc, vc = b['kc'][i], b['vc'][i]
        K.gemm_qkv_rope(xf, Lf['qkv_w'], self.rope, b['pos_suf'],
                        b['ex_q'].view(Ss, -1), kc.view(T, D)[S:],
                        vc[:, :, S:], cfg.heads, D,
                        rownorm_eps=cfg.rms_eps, row_group=Ss,
                        row_group_stride=T, v_ld=T)
        # the attention leaves most CUs idle: its extra workgroups pull the
        # next three GEMMs' weights into the memory-side cache meanwhile
        K.mqa_attention(b['ex_q'], kc[:, :S + Ss], vc, b['ex_ctx'],
                        kgrp=b['kgrp'], qgrp=b['qgrp_suf'], v_transposed=True,
                        o_frag=ctxf, o_row_major=False,
                        prefetch=self._prefetch_list(i),
                        prefetch_place=self.prefetch_place)
        K.gemm(ctxf, Lf['o_w'], out=x, residual=x, c_frag=xf)
        K.gemm_geglu(xf, Lf['gate_w'], Lf['up_w'], out=b['ex_h'],
                     rownorm_eps=cfg.rms_eps, c_frag=hf)
        K.gemm(hf, Lf['down_w'], out=x, residual=x, c_frag=xf)

    def _prefetch_list(self, i):
        """The weights expert layer i's attention prefetches: its O, gate,
        up and down weights and the next layer's Q|K|V (layer 0's after the
        last: the next Euler step starts there), or None when prefetching
        is off."""
        if not self.prefetch:
            return None
        n = (i + 1) % len(self.exp_f)
        Lf, Ln = self.exp_f[i], self.exp_f[n]
        out = [Lf['o_w'], Lf['gate_w'], Lf['up_w'], Lf['down_w'], Ln['qkv_w']]
        if self.prefetch_kv:
            # the next layer's key / value cache (one sample at bs=1) into
            # the memory-side cache
            b = self._bufs[1]
            out += [b['kc'][n], b['vc'][n]]
        return out

    def _expert_layer_pi0(self, b, B, i, L):
        if self._frag_ok(B):
            return self._expert_layer_pi0_frag(b, i, L)
        cfg = self.cfg
        S, Ss, D, hid = cfg.prefix_len, cfg.suffix_len, cfg.head_dim, cfg.exp_hidden
        T = self.kv_len
        x = b['ex_x'].view(B * Ss, hid)
        kc, vc = b['kc'][i], b['vc'][i]
        K.gemm_qkv_rope(x, L['qkv_w'], self.rope, b['pos_suf'],
                        b['ex_q'].view(B * Ss, -1), kc.view(B * T, D)[S:],
                        vc[:, :, S:], cfg.heads, D,
                        rownorm_eps=cfg.rms_eps, row_group=Ss,
                        row_group_stride=T, v_ld=T)
        K.mqa_attention(b['ex_q'], kc[:, :S + Ss], vc, b['ex_ctx'],
                        kgrp=b['kgrp'], qgrp=b['qgrp_suf'], v_transposed=True)
        K.gemm(b['ex_ctx'].view(B * Ss, -1), L['o_w'], out=x, residual=x)
        K.gemm_geglu(x, L['gate_w'], L['up_w'], out=b['ex_h'],
                     rownorm_eps=cfg.rms_eps)
        K.gemm(b['ex_h'], L['down_w'], out=x, residual=x)

    def _fold_ok(self, B, rtc):
        """PI0.5 runs its adaptive RMSNorms folded into the GEMMs at bs=1
        (per-position styles of the prefix RTC method keep the norm
        kernels)."""
        return (self.cfg.pi05 and self.fold_adarms and self.fold is not None
                and self._frag_ok(B) and rtc != 'prefix')

    def _expert_layer_pi05_fused(self, b, i, step):
        """_expert_layer_pi05 at bs=1 with the adaptive RMSNorms folded in:
        the Q|K|V and gate/up GEMMs read the raw stream x (fragment-major),
        scale its columns by 1 + scale and its rows by the RMS factor and
        add shift @ W^T; the O and down epilogues multiply by the style's
        gate before the residual add (condition_gemma.py:126-145, 319-337)."""
        cfg = self.cfg
        S, Ss, D, hid = cfg.prefix_len, cfg.suffix_len, cfg.head_dim, cfg.exp_hidden
        T = self.kv_len
        Lf, fz = self.exp_f[i], self.fold[i]
        x = b['ex_x'].view(Ss, hid)
        xf = b['ex_xf'].rows(Ss)
        ctxf, hf = b['ex_ctxf'].rows(Ss), b['ex_hf'].rows(Ss)
        kc, vc = b['kc'][i], b['vc'][i]
        sa, sp = self.styles[step, 2 * i], self.styles[step, 2 * i + 1]
        K.gemm_qkv_rope(xf, Lf['qkv_w'], self.rope, b['pos_suf'],
                        b['ex_q'].view(Ss, -1), kc.view(T, D)[S:],
                        vc[:, :, S:], cfg.heads, D, rownorm_eps=cfg.rms_eps,
                        row_group=Ss, row_group_stride=T, v_ld=T,
                        a_scale=sa[:hid], bias_f32=fz['qkv'][step])
        K.mqa_attention(b['ex_q'], kc[:, :S + Ss], vc, b['ex_ctx'],
                        kgrp=b['kgrp'], qgrp=b['qgrp_suf'], v_transposed=True,
                        o_frag=ctxf, o_row_major=False,
                        prefetch=self._prefetch_list(i),
                        prefetch_place=self.prefetch_place)
        K.gemm(ctxf, Lf['o_w'], out=x, residual=x,
               gate=sa[2 * hid:].view(1, hid), gate_group=Ss, c_frag=xf)
        K.gemm_geglu(xf, Lf['gate_w'], Lf['up_w'], out=b['ex_h'],
                     rownorm_eps=cfg.rms_eps, c_frag=hf, a_scale=sp[:hid],
                     bias_f32=fz['gate'][step], bias2_f32=fz['up'][step])
        K.gemm(hf, Lf['down_w'], out=x, residual=x,
               gate=sp[2 * hid:].view(1, hid), gate_group=Ss, c_frag=xf)

    def _expert_layer_pi05(self, b, B, i, L, step, rtc=None):
        cfg = self.cfg
        pf = None
        if self._frag_ok(B):
            L = self.exp_f[i]  # fragment-major weights for the skinny GEMMs
            pf = self._prefetch_list(i)
        S, Ss, D, hid = cfg.prefix_len, cfg.suffix_len, cfg.head_dim, cfg.exp_hidden
        T = self.kv_len
        x = b['ex_x'].view(B * Ss, hid)
        xn, gate = b['ex_xn'].view(B * Ss, hid), b['ex_gate'].view(B * Ss, hid)
        kc, vc = b['kc'][i], b['vc'][i]
        st = self.styles[step]
        # prefix RTC: locked positions are conditioned on time 0
        lk = ({'lock': b['rtc_lock'], 'lock_period': Ss}
              if rtc == 'prefix' else {})
        K.adarms_norm(x, st[2 * i:2 * i + 1], out=xn, gate_out=gate,
                      eps=cfg.rms_eps,
                      style_locked=self.styles0[2 * i] if lk else None, **lk)
        K.gemm_qkv_rope(xn, L['qkv_w'], self.rope, b['pos_suf'],
                        b['ex_q'].view(B * Ss, -1), kc.view(B * T, D)[S:],
                        vc[:, :, S:], cfg.heads, D, row_group=Ss,
                        row_group_stride=T, v_ld=T)
        K.mqa_attention(b['ex_q'], kc[:, :S + Ss], vc, b['ex_ctx'],
                        kgrp=b['kgrp'], qgrp=b['qgrp_suf'], v_transposed=True,
                        prefetch=pf, prefetch_place=self.prefetch_place)
        K.gemm(b['ex_ctx'].view(B * Ss, -1), L['o_w'], out=x, residual=x,
               gate=gate)
        K.adarms_norm(x, st[2 * i + 1:2 * i + 2], out=xn, gate_out=gate,
                      eps=cfg.rms_eps,
                      style_locked=self.styles0[2 * i + 1] if lk else None,
                      **lk)
        K.gemm_geglu(xn, L['gate_w'], L['up_w'], out=b['ex_h'])
        K.gemm(b['ex_h'], L['down_w'], out=x, residual=x, gate=gate)

    def transformer_decoder(self, b, B, rtc=None):
        """The Euler loop of the action expert
        (pi05_flowmatching_inference.py:155-312 / pi0_flowmatching.py:
        642-649, 787-831): suffix embedding, expert layers against the
        cached prefix K/V, final norm + action_out_proj + Euler update fused
        in one GEMM epilogue.  ``rtc``: None, 'prefix', 'guidance' or
        'guidance_vjp' (real-time chunking, pi0_flowmatching.py:651-700; see
        fluxvla_amd.rtc; the last runs fluxvla_amd.vjp's loop)."""
        if rtc == 'guidance_vjp':
            return self._vjp_engine().decoder(b, B)
        cfg = self.cfg
        Ss, na, hid = cfg.suffix_len, cfg.n_action_steps, cfg.exp_hidden
        x3 = b['ex_x']
        xt_b = b['xt_bf16'].view(B * na, -1)
        fr = self._frag_ok(B)
        if cfg.pi05:
            w_in = self.act_in_f if fr else self.act_in['w']
        else:
            # the state row of each sample's constant mlp_out residual
            K.gemm(b['states'], self.state['w'], out=b['suf_res'],
                   bias=self.state['b'], row_group=1, row_group_stride=Ss)
            w_mi = self.mlp_in_x_f if fr else self.mlp_in_x
            w_mo = self.mlp_out_f if fr else self.mlp_out['w']
            h = b['suf_h']  # row 0 of each sample (the state row) stays 0
        fused = self._fold_ok(B, rtc)
        for step in range(len(self.times)):
            if cfg.pi05:
                K.gemm(xt_b, w_in, out=x3.view(B * Ss, hid),
                       bias=self.act_in['b'],
                       c_frag=b['ex_xf'].rows(Ss) if fused else None)
            else:
                # prefix RTC: locked positions take the time-0 embedding
                lk = ({'rtc_lock': b['rtc_lock'], 'rtc_period': na,
                       'bias_f32_locked': self.step_bias0}
                      if rtc == 'prefix' else {})
                K.gemm(xt_b, w_mi, out=h[1:], bias_f32=self.step_bias[step],
                       act=ACT_SILU, row_group=na, row_group_stride=Ss, **lk)
                K.gemm(h, w_mo, out=x3.view(B * Ss, hid),
                       residual=b['suf_res'],
                       c_frag=b['ex_xf'].rows(Ss) if fr else None)
            for i, L in enumerate(self.exp['layers']):
                if fused:
                    self._expert_layer_pi05_fused(b, i, step)
                elif cfg.pi05:
                    self._expert_layer_pi05(b, B, i, L, step, rtc)
                else:
                    self._expert_layer_pi0(b, B, i, L)
            # one Euler GEMM for the batch: the action rows of every sample
            # (behind its state row for PI0: A's rows in groups of na)
            lead = Ss - na
            a = x3[:, lead:]
            xt, xtb = b['xt'].view(B * na, -1), b['xt_bf16'].view(B * na, -1)
            w_out = self.act_out_f if fr else self.act_out['w']
            if fused:
                K.gemm_euler(a, w_out, self.act_out['b'], xt, self.dt, xt_bf16=xtb,
                             rownorm_eps=cfg.rms_eps, bias_f32=self.fold_out[step],
                             a_scale=self.styles[step, -1, :hid],
                             **self._euler_rtc(b, B, step, rtc))
                continue
            if cfg.pi05:
                xn = b['ex_xn'][:, lead:]
                st = self.styles[step, -1:]
                lk = ({'style_locked': self.styles0[-1],
                       'lock': b['rtc_lock'], 'lock_period': na}
                      if rtc == 'prefix' else {})
                K.adarms_norm(a, st, out=xn, eps=cfg.rms_eps, **lk)
                a, rn = xn, None
            else:
                rn = cfg.rms_eps
            K.gemm_euler(a, w_out, self.act_out['b'], xt, self.dt, xt_bf16=xtb,
                         rownorm_eps=rn, **self._euler_rtc(b, B, step, rtc))

    def _euler_rtc(self, b, B, step, rtc):
        """Real-time chunking arguments of the batch's Euler GEMM (row m is
        action step m % n_action_steps of its sample)."""
        na = self.cfg.n_action_steps
        prev = b['rtc_prev'].view(B * na, -1)
        if rtc == 'prefix':
            return {'rtc_lock': b['rtc_lock'], 'rtc_period': na, 'rtc_prev': prev}
        if rtc == 'guidance':
            return {'rtc_period': na, 'rtc_prev': prev,
                    'rtc_cw': b['rtc_cw'][step],
                    'rtc_omt': self._rtc_omt[step]}
        return {}

    def _vjp_engine(self):
        """The VJP step of guidance with use_vjp (fluxvla_amd.vjp), built on
        first use: transposed weights and saved-activation buffers."""
        if self._vjp is None:
            from .vjp import ExpertVJP
            self._vjp = ExpertVJP(self)
        return self._vjp

    def _run(self, B, rtc=None):
        b = self._buffers(B)
        self.vision_encoder(b, B)
        self.transformer_encoder(b, B)
        self.transformer_decoder(b, B, rtc)

    # -- request staging (_triton_forward, :486-512) ---------------------------
    @torch.no_grad()
    def _stage(self, b, images, lang_tokens, states, img_masks, lang_masks,
               noise):
        cfg = self.cfg
        B = images.shape[0]
        dev = self.device
        b['images'].copy_(images, non_blocking=True)
        L = lang_tokens.shape[1]
        if L > cfg.max_prompt_len:
            # ProcessPrompts pads to its max_len (180 by default): padding
            # past the buffer's prompt length carries no keys and is dropped
            P = cfg.max_prompt_len
            if lang_masks is None or bool(lang_masks[:, P:].any()):
                raise ValueError(f'prompt of {L} tokens exceeds '
                                 f'max_prompt_len={P}')
            lang_tokens, lang_masks, L = (lang_tokens[:, :P],
                                          lang_masks[:, :P], P)
        b['ids'].zero_()
        b['ids'][:, :L].copy_(lang_tokens, non_blocking=True)
        if img_masks is None:
            img_masks = torch.ones(B, cfg.n_views, dtype=torch.bool,
                                   device=dev)
        if lang_masks is None:
            lang_masks = torch.ones(B, L, dtype=torch.bool, device=dev)
        lm = torch.zeros(B, cfg.max_prompt_len, dtype=torch.bool, device=dev)
        lm[:, :L] = lang_masks.to(dev).bool()
        pad = prefix_pad_mask(img_masks.to(dev), lm, cfg.num_patches)
        kgrp, qg_pre, qg_suf, pos_pre, pos_suf = attention_groups(
            pad, suffix_att_pattern(cfg))
        b['kgrp'].copy_(kgrp)
        b['qgrp_pre'].copy_(qg_pre)
        b['qgrp_suf'].copy_(qg_suf)
        b['pos_pre'].copy_(pos_pre.view(-1))
        b['pos_suf'].copy_(pos_suf.view(-1))
        if not cfg.pi05:
            b['states'].copy_(states.to(dev, BF16), non_blocking=True)
        b['xt'].copy_(noise, non_blocking=True)
        b['xt_bf16'].copy_(noise, non_blocking=True)

    def _stage_rtc(self, b, rtc, prev, prefix_len, rtc_config):
        """Real-time chunking inputs: the previous chunk (zero rows past its
        length), and either the locked prefix length with the locked rows of
        x_t replaced (prefix, pi0_flowmatching.py:651-669) or the per-step
        guidance weights (guidance, :671-700)."""
        if rtc is None:
            return
        cfg, na = self.cfg, self.cfg.n_action_steps
        prev = R.pad_prev_actions(prev.to(self.device, torch.float32),
                                  cfg.max_action_dim, cfg.ori_action_dim)
        B, L = b['xt'].shape[0], prev.shape[1]
        if prev.shape[0] != B:
            raise ValueError(f'prev_actions has batch {prev.shape[0]}, '
                             f'the request {B}')
        if rtc == 'prefix':
            lock = min(prefix_len, na)
            if L < lock:
                raise ValueError(f'prefix_len {prefix_len} needs {lock} rows '
                                 f'of prev_actions, got {L}')
            b['rtc_prev'].zero_()
            b['rtc_prev'][:, :lock].copy_(prev[:, :lock])
            b['rtc_lock'].fill_(lock)
            b['xt'][:, :lock].copy_(prev[:, :lock])
            b['xt_bf16'][:, :lock].copy_(prev[:, :lock])
        else:
            if L > na:
                raise ValueError(f'prev_actions has {L} rows, the chunk {na}')
            b['rtc_prev'].zero_()
            b['rtc_prev'][:, :L].copy_(prev)
            if rtc == 'guidance_vjp':
                w, gw = R.guidance_vjp_tables(self.times, na, prefix_len, L,
                                              rtc_config)
                b['rtc_w'].copy_(w)
                b['rtc_gw'].copy_(gw)
            else:
                b['rtc_cw'].copy_(R.guidance_cw(self.times, self.dt, na,
                                                prefix_len, L, rtc_config))

    def _capture(self, B, rtc=None):
        g = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            self._run(B, rtc)  # warm-up on the capture stream
            torch.cuda.synchronize(self.device)
            g.capture_begin()
            self._run(B, rtc)
            g.capture_end()
        torch.cuda.current_stream(self.device).wait_stream(stream)
        torch.cuda.synchronize(self.device)
        return g

    @torch.no_grad()
    def predict_action(self, images, lang_tokens, states, img_masks=None,
                       lang_masks=None, past_key_values=None, noise=None,
                       prev_actions=None, prefix_len: int = 0,
                       rtc_config: dict = None, *args, **kwargs):
        """The reference signature (pi0_flowmatching.py:702-715), real-time
        chunking included: with prev_actions, prefix_len > 0 and rtc_config
        the loop is the 'prefix' (default) or 'guidance' method, the latter
        with rtc_config['use_vjp'] pulled back through the expert."""
        cfg = self.cfg
        B = images.shape[0]
        if B > self.max_batch:
            raise ValueError(f'batch {B} > max_batch {self.max_batch}')
        if noise is None:
            noise = torch.randn(B, cfg.n_action_steps, cfg.max_action_dim,
                                device=self.device)
        rtc = R.select_method(prev_actions, prefix_len, rtc_config)
        b = self._buffers(B)

        def stage():
            self._stage(b, images, lang_tokens, states, img_masks, lang_masks,
                        noise)
            self._stage_rtc(b, rtc, prev_actions, prefix_len, rtc_config)

        stage()
        if self.use_graph:
            key = B if rtc is None else (B, rtc)
            g = self._graphs.get(key)
            if g is None:
                g = self._graphs[key] = self._capture(B, rtc)
                stage()
            g.replay()
        else:
            self._run(B, rtc)
        out = b['xt'].clone()
        if self.check_merge:
            # waits for the chunk; raises if an in-launch attention merge
            # stopped waiting (the chunk is then wrong) and clears its
            # counters for the next call
            K.attention_check(self.device)
        return out
