"""Drop-in for the pipeline functions of the reference's fused PI0.5 model
(fluxvla/models/vlas/pi05_flowmatching_inference.py:22-326): the same
function names and signatures, the same ``weights`` keys (the dicts the
prepare_triton hooks of hooks.py return) and ``buffers`` keys
(``init_buffers``, after ``_init_buffers`` :356-442), the same op order.

What differs from the reference file, and why:

* attention: the reference's three-step form (``matmul_abT_scale`` ->
  ``softmax_kernel_masklen`` / ``softmax_kernel_prefix_suffix`` ->
  ``matmul_attn_v``, :101-141, :194-242) becomes one fused HIP attention
  call per layer with the same masking: prefix keys past
  ``valid_encoder_len`` are hidden from every query, suffix keys are seen by
  every suffix query.  The key-visibility vector is built on the device
  from ``valid_encoder_len`` (no host sync, capture-safe);
* the Euler state: ``diffusion_noise.add_(action, alpha=-1/num_steps)`` in
  bf16 (:311-312) becomes the action_out_proj GEMM's fused update of an
  fp32 state ``diffusion_noise_f32`` with its bf16 mirror in
  ``diffusion_noise`` (the reference's PyTorch path keeps x_t in fp32,
  pi0_flowmatching.py:718-720; callers stage both);
* RoPE tables are whatever the caller stages in ``encoder_rope_weights`` /
  ``decoder_rope_weights`` (bf16 interleaved (cos, sin) rows, one per
  query row) -- ``rope_rows`` builds them.  The reference stages the
  decoder rows from position ``prefix_len - 1`` (:455-459); the PyTorch
  path (pi0_flowmatching.py:817-819), which ``rope_rows`` follows, starts
  at ``valid_encoder_len``.
"""
import math

import torch

from . import atomic_ops as A
from . import kernels as K
from .weight_layout import as_nk

INT32_MAX = 2**31 - 1
BF16 = torch.bfloat16


def vision_encoder(weights, buffers, num_views, num_vit_layers=27):
    """SigLIP over the staged views into ``vision_x`` (:22-66)."""
    num_patches = buffers['vision_x'].shape[1]
    vit_hidden = buffers['vision_x'].shape[2]
    vit_intermediate = buffers['vision_hidden'].shape[2]
    vit_num_heads = buffers['vit_num_heads']
    vit_head_dim = vit_hidden // vit_num_heads
    patch_size = weights['vision_patch_embedding_w'].shape[0]
    grid_size = int(math.isqrt(num_patches))
    A.conv2d_embed_res(buffers['observation_images_normalized'],
                       weights['vision_patch_embedding_w'],
                       weights['vision_patch_embedding_b'],
                       weights['vision_position_embedding'], buffers['vision_x'],
                       grid_size, patch_size, num_patches, vit_hidden)
    x = buffers['vision_x']
    for i in range(num_vit_layers):
        A.layer_norm_QKV_matmul_bias(
            x, weights['vision_pre_attn_norm_w'][i],
            weights['vision_pre_attn_norm_b'][i],
            weights['vision_attn_qkv_w'][i], weights['vision_attn_qkv_b'][i],
            buffers['vision_QKV'], buffers['vision_x_norm'], num_patches,
            vit_hidden, 3 * vit_hidden, eps=buffers['vit_eps'])
        K.mha_packed_qkv(buffers['vision_QKV'].view(-1, 3 * vit_hidden),
                         buffers['vision_ctx'].view(-1, vit_hidden),
                         num_views, num_patches, vit_num_heads, vit_head_dim)
        A.matmul_bias_res(buffers['vision_ctx'], weights['vision_attn_o_w'][i],
                          weights['vision_attn_o_b'][i], x, x, None,
                          num_patches, vit_hidden)
        A.layer_norm_matmul_bias_gelu(
            x, weights['vision_pre_ffn_norm_w'][i],
            weights['vision_pre_ffn_norm_b'][i], weights['vision_ffn_up_w'][i],
            weights['vision_ffn_up_b'][i], buffers['vision_hidden'],
            buffers['vision_x_norm'], num_patches, vit_hidden,
            vit_intermediate, eps=buffers['vit_eps'])
        A.matmul_split_k_bias_res(buffers['vision_hidden'],
                                  weights['vision_ffn_down_w'][i],
                                  weights['vision_ffn_down_b'][i], x, x, None,
                                  num_patches, vit_intermediate, vit_hidden)


def _key_groups(buffers, encoder_seq_len):
    """kgrp over [prefix | suffix] keys: 0 for prefix keys below
    valid_encoder_len and for every suffix key, INT32_MAX for the padded
    prefix tail; every query has group 0 (bidirectional prefix, PI0.5 suffix
    sees all)."""
    kg = buffers['attn_kgrp']
    idx = buffers['attn_key_index']
    torch.where(idx[:encoder_seq_len] < buffers['valid_encoder_len'],
                buffers['attn_zero'], buffers['attn_hidden'],
                out=kg[:encoder_seq_len])


def transformer_encoder(weights, buffers, encoder_seq_len,
                        num_encoder_layers=18):
    """Projector into the image rows of ``encoder_x``, then the Gemma-2B
    layers filling ``encoder_K`` / ``encoder_V`` rows [0, encoder_seq_len)
    (:69-152); the last layer stops after its K/V as in the reference."""
    hid = buffers['encoder_x'].shape[1]
    n_img = buffers['vision_x'].shape[0] * buffers['vision_x'].shape[1]
    vh = buffers['vision_x'].shape[2]
    hd = buffers['encoder_K'].shape[2]
    heads = buffers['encoder_Q'].shape[0] // encoder_seq_len
    A.layer_norm_matmul_bias(
        buffers['vision_x'], weights['vision_final_norm_w'],
        weights['vision_final_norm_b'],
        weights['encoder_multi_modal_projector_w'],
        weights['encoder_multi_modal_projector_b'],
        buffers['encoder_x'][:n_img], buffers['vision_x_norm'], n_img, vh,
        hid, eps=buffers['vit_eps'])
    _key_groups(buffers, encoder_seq_len)
    kgrp = buffers['attn_kgrp'][:encoder_seq_len].view(1, -1)
    qgrp = buffers['attn_qgrp'][:encoder_seq_len].view(1, -1)
    Q = buffers['encoder_Q'].view(1, encoder_seq_len, heads, hd)
    for i in range(num_encoder_layers):
        A.rms_matmul_qkv_rope(
            buffers['encoder_x'], weights['encoder_attn_qkv_w'][i],
            buffers['encoder_rope_weights'], buffers['encoder_Q'],
            buffers['encoder_K'][i, :encoder_seq_len],
            buffers['encoder_V'][i, :encoder_seq_len],
            buffers['encoder_x_norm'], hidden_dim=hid, head_dim=hd,
            num_kv_heads=heads)
        if i == num_encoder_layers - 1:
            break
        K.mqa_attention(Q, buffers['encoder_K'][i, :encoder_seq_len][None],
                        buffers['encoder_V'][i, :encoder_seq_len][None],
                        buffers['encoder_ctx_buf'].view(1, encoder_seq_len,
                                                        heads, hd),
                        kgrp=kgrp, qgrp=qgrp)
        A.matmul_res(buffers['encoder_ctx_buf'].view(-1, heads * hd),
                     weights['encoder_attn_o_w'][i], buffers['encoder_x'],
                     in_features=heads * hd, out_features=hid)
        A.rms_matmul_gate(buffers['encoder_x'], weights['encoder_ffn_gate_w'][i],
                          weights['encoder_ffn_up_w'][i], buffers['encoder_hidden'],
                          buffers['encoder_x_norm'], hidden_dim=hid,
                          intermediate_dim=buffers['encoder_hidden'].shape[1])
        A.matmul_res(buffers['encoder_hidden'], weights['encoder_ffn_down_w'][i],
                     buffers['encoder_x'],
                     in_features=buffers['encoder_hidden'].shape[1],
                     out_features=hid)


def transformer_decoder(weights, buffers, encoder_seq_len,
                        num_decoder_layers=18, num_steps=10):
    """The 10-step Euler loop of the adaRMS action expert against the cached
    prefix (:155-312)."""
    dec, dh = buffers['decoder_x'].shape
    hd = buffers['encoder_K'].shape[2]
    heads = buffers['decoder_q_buf'].shape[0] // dec
    di = buffers['decoder_hidden'].shape[1]
    total = encoder_seq_len + dec
    kgrp = buffers['attn_kgrp'][:total].view(1, -1)
    qgrp = buffers['attn_qgrp'][:dec].view(1, -1)
    Q = buffers['decoder_q_buf'].view(1, dec, heads, hd)
    for step in range(num_steps):
        A.matmul_bias_silu(weights['decoder_time_embeds'][step].view(1, -1),
                           weights['decoder_time_mlp_in_w'],
                           weights['decoder_time_mlp_in_b'],
                           buffers['decoder_x_buf'][:1], in_features=dh,
                           out_features=dh)
        A.matmul_bias_silu(buffers['decoder_x_buf'][:1],
                           weights['decoder_time_mlp_out_w'],
                           weights['decoder_time_mlp_out_b'],
                           buffers['decoder_time_emb'][:1], in_features=dh,
                           out_features=dh)
        A.matmul_bias_small(buffers['diffusion_noise'],
                            weights['decoder_action_in_proj_w'],
                            weights['decoder_action_in_proj_b'],
                            buffers['decoder_x'], in_features=32,
                            out_features=dh)
        for i in range(num_decoder_layers):
            A.adarms_norm_style_proj(
                buffers['decoder_x'], buffers['decoder_time_emb'],
                weights['decoder_pre_attn_norm_mod_w'][i],
                weights['decoder_pre_attn_norm_mod_b'][i],
                buffers['x_normed_buf'], buffers['gate_buf'],
                buffers['decoder_style'], hidden_dim=dh, style_dim=3 * dh)
            A.matmul_qkv_rope(
                buffers['x_normed_buf'], weights['decoder_attn_qkv_w'][i],
                buffers['decoder_rope_weights'], buffers['decoder_q_buf'],
                buffers['encoder_K'][i, encoder_seq_len:total],
                buffers['encoder_V'][i, encoder_seq_len:total],
                hidden_dim=dh, head_dim=hd, num_kv_heads=heads)
            K.mqa_attention(Q, buffers['encoder_K'][i, :total][None],
                            buffers['encoder_V'][i, :total][None],
                            buffers['decoder_ctx_buf'].view(1, dec, heads, hd),
                            kgrp=kgrp, qgrp=qgrp)
            A.matmul_res_gate(buffers['decoder_ctx_buf'].view(-1, heads * hd),
                              weights['decoder_attn_o_w'][i],
                              buffers['decoder_x'], buffers['gate_buf'],
                              in_features=heads * hd, out_features=dh)
            A.adarms_norm_style_proj(
                buffers['decoder_x'], buffers['decoder_time_emb'],
                weights['decoder_pre_ffn_norm_mod_w'][i],
                weights['decoder_pre_ffn_norm_mod_b'][i],
                buffers['x_normed_buf'], buffers['gate_buf'],
                buffers['decoder_style'], hidden_dim=dh, style_dim=3 * dh)
            A.matmul_gate(buffers['x_normed_buf'], weights['decoder_ffn_gate_w'][i],
                          weights['decoder_ffn_up_w'][i], buffers['decoder_hidden'],
                          in_features=dh, intermediate_dim=di)
            A.matmul_res_gate(buffers['decoder_hidden'],
                              weights['decoder_ffn_down_w'][i],
                              buffers['decoder_x'], buffers['gate_buf'],
                              in_features=di, out_features=dh)
        A.adarms_norm_style_proj(
            buffers['decoder_x'], buffers['decoder_time_emb'],
            weights['decoder_final_norm_mod_w'],
            weights['decoder_final_norm_mod_b'], buffers['x_normed_buf'],
            buffers['gate_buf'], buffers['decoder_style'], hidden_dim=dh,
            style_dim=3 * dh)
        # action_out_proj + Euler update of the fp32 state (bf16 mirror in
        # diffusion_noise, the next step's action_in input)
        K.gemm_euler(buffers['x_normed_buf'],
                     as_nk(weights['decoder_action_out_proj_w']),
                     weights['decoder_action_out_proj_b'],
                     buffers['diffusion_noise_f32'], -1.0 / num_steps,
                     xt_bf16=buffers['diffusion_noise'])


def pi05_model(weights, buffers, num_views, encoder_seq_len, num_vit_layers=27,
               num_encoder_layers=18, num_decoder_layers=18, num_steps=10):
    """The whole chunk (:315-326); every op enqueues on the current stream,
    nothing allocates once the buffers exist, so the call is capturable in
    one HIP graph as in the reference (:463-484)."""
    vision_encoder(weights, buffers, num_views, num_vit_layers)
    transformer_encoder(weights, buffers, encoder_seq_len, num_encoder_layers)
    transformer_decoder(weights, buffers, encoder_seq_len, num_decoder_layers,
                        num_steps)


def init_buffers(num_views, encoder_seq_len, decoder_seq_len, num_kv_layers,
                 device='cuda', vit_image_size=224, vit_num_patches=256,
                 vit_hidden=1152, vit_intermediate=4304, vit_num_heads=16,
                 vit_eps=1e-6, enc_hidden=2048, enc_intermediate=16384,
                 dec_hidden=1024, dec_intermediate=4096, head_dim=256,
                 num_heads=8, action_dim=32):
    """The reference's buffer set (_init_buffers, :356-442: same keys and
    shapes) plus what the fused attention and the fp32 Euler state use
    (``vision_ctx``, ``encoder_ctx_buf`` / ``decoder_ctx_buf`` as the
    attention outputs, the key-visibility vectors, ``diffusion_noise_f32``)
    and the SigLIP geometry entries ``vit_num_heads`` / ``vit_eps``."""
    nv, enc, dec = num_views, encoder_seq_len, decoder_seq_len
    bf = dict(dtype=BF16, device=device)

    def z(*s, **kw):
        return torch.zeros(*s, **(kw or bf))
    i32 = dict(dtype=torch.int32, device=device)
    return {
        'observation_images_normalized': z(nv, vit_image_size, vit_image_size, 3),
        'vision_x': z(nv, vit_num_patches, vit_hidden),
        'vision_x_norm': z(nv, vit_num_patches, vit_hidden),
        'vision_QKV': z(nv, vit_num_patches, 3 * vit_hidden),
        'vision_ctx': z(nv, vit_num_patches, vit_hidden),
        'vision_hidden': z(nv, vit_num_patches, vit_intermediate),
        'vision_x_split_k_buf': z(nv * vit_num_patches * vit_hidden * 4,
                                  dtype=torch.float32, device=device),
        'encoder_rope_weights': z(enc, head_dim),
        'encoder_x': z(enc, enc_hidden),
        'encoder_x_norm': z(enc, enc_hidden),
        'encoder_K': z(num_kv_layers, enc + dec, head_dim),
        'encoder_V': z(num_kv_layers, enc + dec, head_dim),
        'encoder_Q': z(enc * num_heads, head_dim),
        'encoder_hidden': z(enc, enc_intermediate),
        'encoder_ctx_buf': z(enc * num_heads, head_dim),
        'valid_encoder_len': z(1, **i32),
        'decoder_rope_weights': z(dec, head_dim),
        'decoder_x': z(dec, dec_hidden),
        'decoder_x_buf': z(dec, dec_hidden),
        'decoder_action_buf': z(dec, action_dim),
        'decoder_time_emb': z(dec, dec_hidden),
        'decoder_style': z(dec, 3 * dec_hidden),
        'decoder_q_buf': z(dec * num_heads, head_dim),
        'decoder_ctx_buf': z(dec * num_heads, head_dim),
        'decoder_hidden': z(dec, dec_intermediate),
        'x_normed_buf': z(dec, dec_hidden),
        'gate_buf': z(dec, dec_hidden),
        'diffusion_noise': z(dec, action_dim),
        'diffusion_noise_f32': z(dec, action_dim, dtype=torch.float32,
                                 device=device),
        'attn_kgrp': z(enc + dec, **i32),
        'attn_qgrp': z(max(enc, dec), **i32),
        'attn_key_index': torch.arange(enc + dec, **i32),
        'attn_zero': torch.zeros((), **i32),
        'attn_hidden': torch.full((), INT32_MAX, **i32),
        'vit_num_heads': vit_num_heads,
        'vit_eps': vit_eps,
    }


def rope_rows(positions, head_dim=256, theta=10000.0):
    """bf16 [len(positions), head_dim] rows of interleaved (cos, sin) pairs
    of position * inv_freq, inv_freq = 1 / theta^(2i / head_dim) in fp32 --
    the reference's table format (:444-456) at the given positions."""
    inv = 1.0 / (theta**(torch.arange(0, head_dim, 2, dtype=torch.float32,
                                      device=positions.device) / head_dim))
    ph = positions.float()[:, None] * inv[None, :]
    return torch.stack([torch.cos(ph), torch.sin(ph)], -1).to(BF16).reshape(
        len(positions), head_dim)


def time_embeds(num_steps, dim=1024, device='cuda'):
    """``decoder_time_embeds`` [num_steps, dim] bf16: the sinusoidal
    embedding of t = 1, 1 + dt, ... (_prepare_adarms_cond, :564-583)."""
    from .pi0_inference import euler_times, sinusoid
    times, _ = euler_times(num_steps)
    return sinusoid(times, dim).to(BF16).to(device)
