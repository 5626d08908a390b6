"""Drop-in counterparts of the PI-path functions of fluxvla/ops/atomic_ops.py
(:34-378) and of ``matmul_bias_cuda`` (fluxvla/ops/cuda/matmul_bias/
matmul_bias.py:19-60): same names, argument order and meaning, each running
the HIP kernels of libfluxvla_amd.so on the current stream and writing into
the caller's preallocated buffers.

Operand conventions:
  * weights mean what the reference's hooks hand its ops: a plain tensor is
    [in_features, out_features] (``W.T``, condition_gemma_inference.py:
    91-105; ``matmul_bias_cuda`` reads N = weight.size(1)) and is transposed
    once on first use (weight_layout.as_nk); the ``NKWeight`` values this
    package's hooks emit (hooks.py) already hold [out, in] and present the
    reference's [in, out] shape; fragment-major and fp8 weights from the
    model's own preparation pass through;
  * Q/K weight columns are pair-interleaved for RoPE (condition_gemma_
    inference.py:46-63), and the Gemma (1 + w) norm scale is folded in;
  * ``rope_weight`` is either the kernels' fp32 [positions, head_dim/2, 2]
    (cos, sin) table (rows = token positions 0..) or the reference's
    interleaved bf16 [positions, head_dim] table (converted once, cached);
  * patch weights are the reference's [kH, kW, C, out] (converted once) or
    the hooks' prepared [out, 3*p*p padded to 8] in (c, ky, kx) order.
Block-size arguments of the Triton wrappers are accepted and ignored: the
HIP kernels choose their own tiling.  The unfused attention trio
(matmul_abT_scale / softmax_kernel_* / matmul_attn_v) is replaced by the
fused ``kernels.mqa_attention``; ``matmul_attn_v`` is kept for callers that
still run the three-step form.
"""
import torch

from . import kernels as _kern
from ._lib import ACT_GELU_TANH, ACT_SILU
from .weight_layout import _cached, as_nk, patch_weight_nk

RMS_EPS = 1e-6


def _rows(x):
    return x.reshape(-1, x.shape[-1])


# ---------------------------------------------------------------------------
# Vision encoder ops
# ---------------------------------------------------------------------------
def conv2d_embed_res(images, patch_w, patch_b, pos_emb, out, grid_size,
                     patch_size, num_patches, vit_hidden):
    """Patch-embedding conv as im2col + GEMM + bias + position embedding
    (atomic_ops.py:34-53).  images: [n_views, H, W, 3] (NHWC, as the
    reference stages them) or [n_views, 3, H, W]."""
    nhwc = images.shape[-1] == 3
    kp = (3 * patch_size * patch_size + 7) // 8 * 8
    w = patch_weight_nk(patch_w, kp)
    patches = _kern.im2col_patches(images, patch_size, kp, channels_last=nhwc)
    _kern.gemm(patches, w, out=_rows(out), bias=patch_b, pos=pos_emb,
               pos_period=num_patches)
    del grid_size, vit_hidden
    return out


def layer_norm_QKV_matmul_bias(x, norm_w, norm_b, qkv_w, qkv_b, out, x_norm,
                               num_patches, vit_hidden, vit_qkv_hidden,
                               eps=1e-6):
    """LayerNorm then packed QKV projection + bias (atomic_ops.py:56-62).
    eps follows the SigLIP config (1e-6); the reference Triton kernel's
    default is 1e-5 (norm_triton_ops.py:97)."""
    _kern.layer_norm(_rows(x), norm_w, norm_b, eps, out=_rows(x_norm))
    _kern.gemm(_rows(x_norm), as_nk(qkv_w), out=_rows(out), bias=qkv_b)
    return out


def AttnMultiKey(QKV, num_patches, vit_num_heads, vit_head_dim, vit_hidden):
    """Per-view bidirectional MHA over packed QKV (atomic_ops.py:65-76)."""
    q2 = _rows(QKV)
    n_views = q2.shape[0] // num_patches
    out = torch.empty(n_views, num_patches, vit_hidden, dtype=QKV.dtype,
                      device=QKV.device)
    _kern.mha_packed_qkv(q2, out.view(-1, vit_hidden), n_views, num_patches,
                     vit_num_heads, vit_head_dim)
    return out


def matmul_bias_res(x, weight, bias, res, out, buf, num_patches, vit_hidden):
    """out = x @ W + bias + res (atomic_ops.py:79-80)."""
    _kern.gemm(_rows(x), as_nk(weight), out=_rows(out), bias=bias,
               residual=_rows(res))
    return out


def layer_norm_matmul_bias_gelu(x, norm_w, norm_b, weight, bias, out, x_norm,
                                num_patches, vit_hidden, vit_intermediate,
                                eps=1e-6):
    """LayerNorm then fc1 + bias + gelu_tanh (atomic_ops.py:83-104)."""
    _kern.layer_norm(_rows(x), norm_w, norm_b, eps, out=_rows(x_norm))
    _kern.gemm(_rows(x_norm), as_nk(weight), out=_rows(out), bias=bias,
               act=ACT_GELU_TANH)
    return out


def matmul_split_k_bias_res(x, weight, bias, res, out, buf, num_patches,
                            vit_intermediate, vit_hidden):
    """fc2 + bias + residual (atomic_ops.py:107-109)."""
    _kern.gemm(_rows(x), as_nk(weight), out=_rows(out), bias=bias,
               residual=_rows(res))
    return out


def layer_norm_matmul_bias(x, norm_w, norm_b, proj_w, proj_b, out, x_norm,
                           num_patches, in_features, out_features, eps=1e-5):
    """LayerNorm then projection + bias (atomic_ops.py:117-149)."""
    _kern.layer_norm(_rows(x), norm_w, norm_b, eps, out=_rows(x_norm))
    _kern.gemm(_rows(x_norm), as_nk(proj_w), out=_rows(out), bias=proj_b)
    return out


# ---------------------------------------------------------------------------
# Gemma ops
# ---------------------------------------------------------------------------
_rope_cache = {}


def _qrows(Q, rows):
    """Q as [tokens, heads * head_dim]: the reference's buffers hold it as
    [tokens * heads, head_dim] (pi05_flowmatching_inference.py:400-401),
    the same memory."""
    if not Q.is_contiguous():
        raise ValueError('Q must be contiguous')
    return Q.view(rows, -1)


def _rope_args(rope_weight, rows, device):
    """(fp32 [positions, hd/2, 2] table, int32 positions 0..rows-1).  A
    reference bf16 table is converted once per (tensor, version) and the
    position vector made once per (rows, device), so repeated calls (and
    graph capture after a warm-up call) allocate nothing."""
    if rope_weight.dtype == torch.float32 and rope_weight.dim() == 3:
        table = rope_weight
    else:  # reference table: interleaved (cos, sin) bf16 [positions, hd]
        # converted once into a cached fp32 copy (refreshed in place when
        # the table changes), like the weights' [out, in] copies
        table = _cached(rope_weight, 'rope', lambda t: t.float().reshape(
            t.shape[0], -1, 2).contiguous())
    if table.shape[0] < rows:
        raise ValueError(f'rope table has {table.shape[0]} positions, need '
                         f'{rows}')
    key = ('pos', rows, torch.device(device))
    pos = _rope_cache.get(key)
    if pos is None:
        pos = _rope_cache[key] = torch.arange(rows, dtype=torch.int32,
                                              device=device)
    return table, pos


def rms_matmul_qkv_rope(x, weight_qkv, rope_weight, Q, K, V, x_norm,
                        hidden_dim, head_dim, num_kv_heads):
    """RMSNorm (no weight: (1 + w) is folded into weight_qkv) fused into the
    QKV GEMM, RoPE on Q and K, split into Q / K / V (atomic_ops.py:155-164).
    ``num_kv_heads`` is the number of query heads, as in the reference's
    call (pi05_flowmatching_inference.py:85-95).  x_norm is not written: the
    normalization never leaves registers."""
    rows = _rows(x).shape[0]
    table, pos = _rope_args(rope_weight, rows, x.device)
    _kern.gemm_qkv_rope(_rows(x), as_nk(weight_qkv), table, pos,
                        _qrows(Q, rows), _rows(K), _rows(V), num_kv_heads,
                        head_dim, rownorm_eps=RMS_EPS)


def matmul_qkv_rope(x_normed, weight_qkv, rope_weight, Q, K, V, hidden_dim,
                    head_dim, num_kv_heads):
    """QKV GEMM + RoPE without a norm (atomic_ops.py:303-311)."""
    rows = _rows(x_normed).shape[0]
    table, pos = _rope_args(rope_weight, rows, x_normed.device)
    _kern.gemm_qkv_rope(_rows(x_normed), as_nk(weight_qkv), table, pos,
                        _qrows(Q, rows), _rows(K), _rows(V), num_kv_heads,
                        head_dim)


def matmul_res(x, weight, out, in_features, out_features):
    """out += x @ W in place (atomic_ops.py:172-188)."""
    o = _rows(out)
    _kern.gemm(_rows(x), as_nk(weight), out=o, residual=o)
    return out


def rms_matmul_gate(x, gate_w, up_w, out, x_norm, hidden_dim,
                    intermediate_dim):
    """RMSNorm fused into the GeGLU dual GEMM (atomic_ops.py:196-201):
    out = gelu_tanh(n(x) @ Wg^T) * (n(x) @ Wu^T); x_norm is not written."""
    _kern.gemm_geglu(_rows(x), as_nk(gate_w), as_nk(up_w), out=_rows(out),
                     rownorm_eps=RMS_EPS)
    return out


def matmul_gate(x, gate_w, up_w, out, in_features, intermediate_dim):
    """GeGLU dual GEMM without a norm (atomic_ops.py:373-378)."""
    _kern.gemm_geglu(_rows(x), as_nk(gate_w), as_nk(up_w), out=_rows(out))
    return out


def matmul_attn_v(x, V, out, head_dim):
    """out = P @ V for the three-step attention form (atomic_ops.py:
    209-221).  V is [keys, head_dim] (K-major for this product), so it is
    transposed once per call; the fused mqa_attention avoids this."""
    vt = V.reshape(-1, head_dim).t().contiguous()
    _kern.gemm(_rows(x), vt, out=_rows(out))
    return out


def matmul_bias_silu(x, weight, bias, out, in_features, out_features):
    """silu(x @ W + b) (atomic_ops.py:229-243)."""
    _kern.gemm(_rows(x), as_nk(weight), out=_rows(out), bias=bias,
               act=ACT_SILU)
    return out


def matmul_bias_small(x, weight, bias, out, in_features, out_features,
                      BLOCK_SIZE_N=32, BLOCK_SIZE_M=32, BLOCK_SIZE_K=32):
    """x @ W + b (atomic_ops.py:251-273)."""
    _kern.gemm(_rows(x), as_nk(weight), out=_rows(out), bias=bias)
    return out


def adarms_norm_style_proj(x, time_emb, mod_w, mod_b, x_normed, gate, style,
                           hidden_dim, style_dim):
    """style = dense(time_emb) (row 0 is the one the norm reads), then
    x_normed = rms(x) * (1 + scale) + shift and gate
    (atomic_ops.py:278-299, norm_triton_ops.py:355-395)."""
    _kern.gemm(_rows(time_emb)[:1], as_nk(mod_w), out=_rows(style)[:1],
               bias=mod_b)
    _kern.adarms_norm(_rows(x), _rows(style)[:1], out=_rows(x_normed),
                  gate_out=_rows(gate), eps=RMS_EPS)


def matmul_res_gate(x, weight, out, gate, in_features, out_features,
                    BLOCK_SIZE_N=32, BLOCK_SIZE_M=32, BLOCK_SIZE_K=128):
    """out += (x @ W) * gate in place (atomic_ops.py:343-365)."""
    o = _rows(out)
    _kern.gemm(_rows(x), as_nk(weight), out=o, residual=o, gate=_rows(gate))
    return out


# ---------------------------------------------------------------------------
# matmul_bias_cuda (cuBLASLt GEMM + bias (+ residual) in the reference)
# ---------------------------------------------------------------------------
def matmul_bias_cuda(inp, weight, bias, out=None, res=None):
    """out = inp @ W + bias (+ res), inp 2-D or 3-D bf16 (matmul_bias.py:
    19-60).  ``weight`` is the reference's [K, N] (a plain tensor, transposed
    once and cached) or an ``NKWeight`` from this package's hooks."""
    orig = inp.shape
    a = inp.reshape(-1, orig[-1])
    w = as_nk(weight)
    if w.shape[1] != a.shape[1]:
        raise ValueError(f'weight of logical shape {tuple(weight.shape)} '
                         f'([K, N]) does not match inp {tuple(orig)}')
    N = w.shape[0]
    if out is None:
        out = torch.empty(*orig[:-1], N, dtype=inp.dtype, device=inp.device)
    _kern.gemm(a, w, out=out.reshape(-1, N), bias=bias,
           residual=None if res is None else res.reshape(-1, N))
    return out
