"""ctypes binding of libfluxvla_amd.so (the C ABI in include/fluxvla_amd.h).

The library is loaded from the package directory.  There is no fallback: if
the shared object is missing or a symbol is absent, importing the kernels
raises, so nothing can silently run a CPU path in its place.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, 'libfluxvla_amd.so')

c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p

FVX_OK = 0
FVX_ERR_NULL = -1
FVX_ERR_SHAPE = -2
FVX_ERR_ALIGN = -3
FVX_ERR_LAUNCH = -4
FVX_ERR_ARG = -5
FVX_ERR_WORKSPACE = -6
FVX_ERR_MERGE = -7

# fvx_gemm_noalloc's static split-K scratch per GPU
GEMM_NOALLOC_SCRATCH_BYTES = 32 << 20

GEMM_PLAIN, GEMM_GEGLU, GEMM_QKV_ROPE, GEMM_EULER = 0, 1, 2, 3
ACT_NONE, ACT_SILU, ACT_GELU_TANH = 0, 1, 2


class GemmDesc(ctypes.Structure):
    """Mirror of ``fvx_gemm_desc``."""
    _fields_ = [
        ('a', c_vp), ('lda', c_i64),
        ('b', c_vp), ('ldb', c_i64),
        ('b2', c_vp),
        ('c', c_vp), ('ldc', c_i64),
        ('m', c_i64), ('n', c_i64), ('k', c_i64),
        ('bias', c_vp),
        ('bias_f32', c_vp),
        ('residual', c_vp), ('ldr', c_i64),
        ('gate', c_vp), ('ldg', c_i64), ('gate_group', c_i64),
        ('pos', c_vp), ('ldp', c_i64), ('pos_period', c_i64),
        ('act', c_i32),
        ('mode', c_i32),
        ('rownorm', c_i32),
        ('out_f32', c_i32),
        ('rownorm_eps', c_f32),
        ('dt', c_f32),
        ('row_group', c_i64), ('row_group_stride', c_i64),
        ('rope', c_vp),
        ('positions', c_vp),
        ('q_out', c_vp), ('ldq', c_i64),
        ('k_out', c_vp), ('ldk', c_i64),
        ('v_out', c_vp), ('ldv', c_i64),
        ('n_q_heads', c_i32), ('head_dim', c_i32),
        ('xt', c_vp), ('ldx', c_i64),
        ('xt_bf16', c_vp), ('ldxb', c_i64),
        ('workspace', c_vp), ('workspace_bytes', c_i64),
        ('split_k', c_i32),
        ('v_transposed', c_i32),
        ('a_frag', c_i32), ('b_frag', c_i32),
        ('c_frag', c_vp),
        ('b_fp8', c_i32),
        ('b_scale', c_vp), ('b2_scale', c_vp),
        ('ss_out', c_vp), ('ss_in', c_vp), ('ss_ld', c_i64), ('ss_parts', c_i32),
        ('a8_out', c_vp), ('a8_out_scale', c_vp), ('a8_out_ld', c_i64), ('a8_out_sld', c_i64),
        ('a8', c_vp), ('a8_scale', c_vp), ('a8_ld', c_i64), ('a8_sld', c_i64),
        ('fp8_act', c_i32),
        ('rtc_lock', c_vp), ('rtc_period', c_i64),
        ('bias_f32_locked', c_vp),
        ('rtc_prev', c_vp), ('ld_prev', c_i64),
        ('rtc_cw', c_vp),
        ('rtc_omt', c_f32),
        ('a_scale', c_vp), ('bias2_f32', c_vp),
        ('ln_csum', c_vp),
        ('a_row_group', c_i64), ('a_row_group_stride', c_i64),
        ('gu_out', c_vp), ('ld_gu', c_i64),
        ('k_t_out', c_vp), ('ld_kt', c_i64),
        ('v_rows_out', c_vp), ('ld_vr', c_i64),
    ]


class AttnDesc(ctypes.Structure):
    """Mirror of ``fvx_attn_desc``."""
    _fields_ = [
        ('q', c_vp), ('q_tok_stride', c_i64), ('q_head_stride', c_i64),
        ('q_zs1', c_i64), ('q_zs2', c_i64),
        ('k', c_vp), ('k_tok_stride', c_i64), ('k_zs1', c_i64),
        ('k_zs2', c_i64),
        ('v', c_vp), ('v_tok_stride', c_i64), ('v_zs1', c_i64),
        ('v_zs2', c_i64),
        ('v_d_stride', c_i64),
        ('o', c_vp), ('o_tok_stride', c_i64), ('o_head_stride', c_i64),
        ('o_zs1', c_i64), ('o_zs2', c_i64),
        ('kgrp', c_vp), ('kgrp_zs1', c_i64),
        ('qgrp', c_vp), ('qgrp_zs1', c_i64),
        ('sq', c_i64), ('sk', c_i64), ('heads', c_i64), ('head_dim', c_i64),
        ('n_problems', c_i64), ('zdiv', c_i64),
        ('scale', c_f32),
        ('kv_splits', c_i32),
        ('workspace', c_vp), ('workspace_bytes', c_i64),
        ('o_frag', c_vp),
        ('prefetch', c_vp * 8), ('prefetch_bytes', c_i64 * 8),
        ('prefetch_tile_bytes', c_i64 * 8),
        ('prefetch_wgs', c_i32),
        ('merge_no_wait', c_i32),
    ]


class ImageDesc(ctypes.Structure):
    """Mirror of ``fvx_image_desc``."""
    _fields_ = [
        ('src', c_vp), ('src_u8', c_i32), ('src_hwc', c_i32),
        ('n', c_i64), ('src_h', c_i64), ('src_w', c_i64),
        ('src_img_stride', c_i64),
        ('dst', c_vp), ('dst_h', c_i64), ('dst_w', c_i64),
        ('dst_img_stride', c_i64),
        ('rh', c_i64), ('rw', c_i64), ('off_y', c_i64), ('off_x', c_i64),
        ('pad_value', c_f32),
        ('filter', c_i32), ('round_u8', c_i32), ('swap_rb', c_i32),
        ('pre_div', c_f32),
        ('mean', c_f32 * 3), ('den', c_f32 * 3),
        ('pad_per_channel', c_i32), ('pad_rgb', c_f32 * 3),
    ]


RESIZE_LINEAR, RESIZE_PIL_BILINEAR = 0, 1


class AttnBwdDesc(ctypes.Structure):
    """Mirror of ``fvx_attn_bwd_desc``."""
    _fields_ = [
        ('q', c_vp), ('q_zs', c_i64),
        ('o', c_vp), ('o_zs', c_i64),
        ('dout', c_vp), ('do_zs', c_i64),
        ('k', c_vp), ('k_zs', c_i64),
        ('v', c_vp), ('v_zs', c_i64),
        ('kt', c_vp), ('kt_ld', c_i64), ('kt_zs', c_i64),
        ('vt', c_vp), ('vt_ld', c_i64), ('vt_zs', c_i64),
        ('refresh_key0', c_i64), ('refresh_n', c_i64),
        ('kgrp', c_vp), ('kgrp_zs', c_i64),
        ('qgrp', c_vp), ('qgrp_zs', c_i64),
        ('stats', c_vp),
        ('dq', c_vp), ('dq_parts', c_i64),
        ('ds_t', c_vp), ('p_t', c_vp), ('ldt', c_i64), ('t_zs', c_i64),
        ('rows', c_i64), ('heads', c_i64), ('head_dim', c_i64),
        ('n_keys', c_i64), ('key0', c_i64), ('n_suffix', c_i64),
        ('n_problems', c_i64),
        ('scale', c_f32),
    ]

# name -> (restype, argtypes); the exact set declared by include/fluxvla_amd.h
SIGNATURES = {
    'fvx_version': (c_i32, []),
    'fvx_last_error': (ctypes.c_char_p, []),
    'fvx_gemm_workspace_bytes': (c_i64, [ctypes.POINTER(GemmDesc)]),
    'fvx_gemm': (c_i32, [ctypes.POINTER(GemmDesc), c_vp]),
    'fvx_gemm_noalloc': (c_i32, [ctypes.POINTER(GemmDesc), c_vp]),
    'fvx_rms_norm_residual':
    (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_f32, c_vp]),
    'fvx_layer_norm': (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_f32,
                               c_vp]),
    'fvx_adarms_norm': (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                                c_i64, c_f32, c_vp]),
    'fvx_adarms_norm_locked': (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_vp,
                                       c_vp, c_i64, c_i64, c_i64, c_i64,
                                       c_f32, c_vp]),
    'fvx_attention_workspace_bytes': (c_i64, [ctypes.POINTER(AttnDesc)]),
    'fvx_attention': (c_i32, [ctypes.POINTER(AttnDesc), c_vp]),
    'fvx_attention_check': (c_i32, [c_vp, c_i64, c_vp]),
    'fvx_im2col_patches': (c_i32, [c_vp, c_i32, c_i32, c_vp, c_i64, c_i64,
                                   c_i64, c_i64, c_i64, c_f32, c_f32, c_vp]),
    'fvx_embed_tokens': (c_i32, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_f32,
                                 c_i64, c_i64, c_vp]),
    'fvx_pack_frag': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp]),
    'fvx_copy_rows': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_i64,
                              c_i64, c_vp]),
    'fvx_resize_normalize': (c_i32, [ctypes.POINTER(ImageDesc), c_vp]),
    # backward ops of guidance RTC with use_vjp
    'fvx_rms_norm_backward': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64,
                                      c_vp, c_vp, c_vp, c_i64, c_vp, c_i64,
                                      c_vp, c_i64, c_i64, c_i64, c_i64, c_f32,
                                      c_vp]),
    'fvx_act_backward': (c_i32, [c_i32, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64,
                                 c_vp, c_i64, c_i64, c_vp]),
    'fvx_geglu_rows': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_i64,
                               c_vp]),
    'fvx_attention_rows_backward': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp,
                                            c_vp, c_vp, c_i64, c_vp, c_vp,
                                            c_i64, c_i64, c_i64, c_i64, c_i64,
                                            c_i64, c_i64, c_f32, c_vp]),
    'fvx_attention_suffix_kv_backward': (c_i32, [c_vp, c_vp, c_i64, c_vp,
                                                 c_i64, c_vp, c_i64, c_vp,
                                                 c_i64, c_vp, c_i64, c_i64,
                                                 c_i64, c_i64, c_vp]),
    'fvx_transpose_bf16': (c_i32, [c_vp, c_i64, c_i64, c_vp, c_i64, c_i64,
                                   c_i64, c_i64, c_i64, c_vp]),
    'fvx_rope_backward': (c_i32, [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64,
                                  c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp,
                                  c_i64, c_i64, c_i64, c_vp]),
    'fvx_attention_backward': (c_i32, [ctypes.POINTER(AttnBwdDesc), c_vp]),
    'fvx_attention_backward_parts': (c_i64, [c_i64]),
    'fvx_rtc_vjp_error': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp,
                                  c_vp, c_i64, c_i64, c_i64, c_i64, c_f32,
                                  c_vp]),
    'fvx_rtc_vjp_update': (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64,
                                   c_vp, c_i64, c_vp, c_vp, c_i64, c_vp,
                                   c_i64, c_i64, c_i64, c_f32, c_f32, c_vp]),
}

ACT_BWD_GEGLU, ACT_BWD_SILU = 0, 1

_lib = None


class FvxError(RuntimeError):
    """A C-ABI entry point returned a non-zero fvx_status."""

    def __init__(self, name, code, message):
        super().__init__(f'{name} failed (status {code}): {message}')
        self.code = code


def load():
    """Load the shared library (once) and bind every declared symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f'{LIB_PATH} is not built; run `python -c "import '
            '__graft_entry__ as g; g.build()"` (hipcc, gfx950) first')
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the export is missing
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(name, *args):
    """Call entry point ``name``; raise FvxError on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != FVX_OK:
        msg = lib.fvx_last_error().decode(errors='replace')
        if rc in (FVX_ERR_SHAPE, FVX_ERR_ARG, FVX_ERR_NULL, FVX_ERR_ALIGN):
            raise ValueError(f'{name}: {msg} (status {rc})')
        raise FvxError(name, rc, msg)
    return rc
