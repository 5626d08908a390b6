"""The C-ABI library loads, exports exactly what include/fluxvla_amd.h
declares, and rejects bad arguments with status codes (no GPU needed: every
check below fails validation before any HIP call is made)."""
import ctypes
import os
import re

import pytest

from fluxvla_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'fluxvla_amd.h')


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(fvx_\w+)\s*\(', text)))


def test_header_matches_binding_table():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.fvx_version() == 1


def test_gemm_desc_layout_matches_c():
    names = [f[0] for f in _lib.GemmDesc._fields_]
    text = open(HEADER).read()
    body = text[text.index('typedef struct fvx_gemm_desc'):]
    body = body[:body.index('} fvx_gemm_desc;')]
    body = re.sub(r'/\*.*?\*/', '', body, flags=re.S)
    c_names = re.findall(r'\*?\s*(\w+)\s*(?:\[\d+\])?\s*[;,]', body)
    assert c_names == names


def test_attn_desc_layout_matches_c():
    names = [f[0] for f in _lib.AttnDesc._fields_]
    text = open(HEADER).read()
    body = text[text.index('typedef struct fvx_attn_desc'):]
    body = body[:body.index('} fvx_attn_desc;')]
    body = re.sub(r'/\*.*?\*/', '', body, flags=re.S)
    c_names = re.findall(r'\*?\s*(\w+)\s*(?:\[\d+\])?\s*[;,]', body)
    assert c_names == names
    # array fields keep their C lengths
    fields = dict(_lib.AttnDesc._fields_)
    assert all(fields[f]._length_ == 8 for f in
               ('prefetch', 'prefetch_bytes', 'prefetch_tile_bytes'))


def _err(lib):
    return lib.fvx_last_error().decode()


def test_gemm_rejects_bad_arguments():
    lib = _lib.load()
    d = _lib.GemmDesc()
    assert lib.fvx_gemm(None, None) == _lib.FVX_ERR_NULL
    assert lib.fvx_gemm(ctypes.byref(d), None) == _lib.FVX_ERR_NULL
    d.a, d.b, d.c = 4096, 8192, 16384
    d.m, d.n, d.k, d.lda, d.ldb, d.ldc = 4, 4, 12, 12, 12, 4
    assert lib.fvx_gemm(ctypes.byref(d), None) == _lib.FVX_ERR_SHAPE
    assert 'multiples of 8' in _err(lib)
    d.k = d.lda = d.ldb = 16
    d.a = 4100
    assert lib.fvx_gemm(ctypes.byref(d), None) == _lib.FVX_ERR_ALIGN
    d.a = 4096
    d.mode = 7
    assert lib.fvx_gemm(ctypes.byref(d), None) == _lib.FVX_ERR_ARG
    d.mode = _lib.GEMM_GEGLU  # needs b2
    assert lib.fvx_gemm(ctypes.byref(d), None) == _lib.FVX_ERR_NULL
    d.mode = _lib.GEMM_QKV_ROPE
    d.rope = d.positions = d.q_out = d.k_out = d.v_out = 4096
    d.n_q_heads, d.head_dim = 8, 256
    assert lib.fvx_gemm(ctypes.byref(d), None) == _lib.FVX_ERR_SHAPE
    assert 'n_q_heads + 2' in _err(lib)


def test_gemm_rejects_periods_past_32_bits():
    # the epilogue divides rows by row_group / gate_group / pos_period /
    # rtc_period in 32 bits, so the host refuses values from 2^31 on
    lib = _lib.load()
    for field in ('row_group', 'gate_group', 'pos_period', 'rtc_period'):
        d = _lib.GemmDesc()
        d.a, d.b, d.c = 4096, 8192, 16384
        d.m, d.n, d.k, d.lda, d.ldb, d.ldc = 4, 8, 16, 16, 16, 8
        setattr(d, field, 1 << 31)
        assert lib.fvx_gemm(ctypes.byref(d), None) == _lib.FVX_ERR_SHAPE, field
        assert '2^31' in _err(lib)


def test_gemm_rejects_bad_layernorm_fold():
    # ln_csum: PLAIN, rownorm, M > 64, sums taken in the K loop (no ss_in),
    # bf16 weights, one K range, nothing handed over
    lib = _lib.load()

    def desc(**kw):
        d = _lib.GemmDesc()
        d.a, d.b, d.c = 4096, 8192, 16384
        d.m, d.n, d.k, d.lda, d.ldb, d.ldc = 128, 64, 64, 64, 64, 64
        d.rownorm, d.rownorm_eps, d.ln_csum = 1, 1e-6, 32768
        for k, v in kw.items():
            setattr(d, k, v)
        return d
    for kw in ({'rownorm': 0}, {'m': 64, 'ldc': 64}, {'ss_in': 65536, 'ss_parts': 1, 'ss_ld': 128},
               {'ss_out': 65536, 'ss_ld': 128}, {'split_k': 2}, {'mode': _lib.GEMM_QKV_ROPE}):
        assert lib.fvx_gemm(ctypes.byref(desc(**kw)), None) == _lib.FVX_ERR_ARG, kw
        assert 'ln_csum' in _err(lib), kw


def test_gemm_explicit_split_without_workspace_is_an_error():
    lib = _lib.load()
    d = _lib.GemmDesc()
    d.a, d.b, d.c = 4096, 8192, 16384
    d.m, d.n, d.k, d.lda, d.ldb, d.ldc = 8, 64, 4096, 4096, 4096, 64
    d.split_k = 8
    assert lib.fvx_gemm_workspace_bytes(ctypes.byref(d)) > 0
    assert lib.fvx_gemm(ctypes.byref(d), None) == _lib.FVX_ERR_WORKSPACE


def test_norm_and_attention_reject_bad_arguments():
    lib = _lib.load()
    assert lib.fvx_rms_norm_residual(None, None, None, None, None, 1, 8,
                                     1e-6, None) == _lib.FVX_ERR_NULL
    assert lib.fvx_rms_norm_residual(4096, None, None, 8192, None, 1, 12,
                                     1e-6, None) == _lib.FVX_ERR_SHAPE
    assert lib.fvx_rms_norm_residual(4096, None, None, 8192, None, 1, 8192,
                                     1e-6, None) == _lib.FVX_ERR_SHAPE
    assert lib.fvx_layer_norm(4096, None, 4096, 4096, 1, 8, 1e-6,
                              None) == _lib.FVX_ERR_NULL
    assert lib.fvx_adarms_norm(4096, 4096, 4096, None, 2, 8, 1, 16, 1e-6,
                               None) == _lib.FVX_ERR_SHAPE
    a = _lib.AttnDesc()
    assert lib.fvx_attention(ctypes.byref(a), None) == _lib.FVX_ERR_NULL
    a.q = a.k = a.v = a.o = 4096
    a.sq, a.sk, a.heads, a.n_problems, a.zdiv = 4, 4, 1, 1, 1
    a.head_dim = 128
    assert lib.fvx_attention(ctypes.byref(a), None) == _lib.FVX_ERR_SHAPE
    a.head_dim = 256
    a.kgrp = 4096
    assert lib.fvx_attention(ctypes.byref(a), None) == _lib.FVX_ERR_ARG
    a.kgrp = 0
    a.sq, a.heads = 1 << 28, 8  # query rows past 32-bit indices
    assert lib.fvx_attention(ctypes.byref(a), None) == _lib.FVX_ERR_SHAPE
    assert '2^31' in _err(lib)


def test_data_movement_rejects_bad_arguments():
    lib = _lib.load()
    assert lib.fvx_im2col_patches(4096, 0, 0, 4096, 1, 224, 224, 14, 580,
                                  1.0, 0.0, None) == _lib.FVX_ERR_SHAPE
    assert lib.fvx_embed_tokens(4096, None, 4096, 1, 8, 8, 1.0, 0, 0,
                                None) == _lib.FVX_ERR_NULL
    assert lib.fvx_copy_rows(4096, 8, 4096, 8, 1, 12, 0, 0,
                             None) == _lib.FVX_ERR_SHAPE


def test_python_layer_raises_value_error_on_status():
    with pytest.raises(ValueError, match='multiples of 8'):
        d = _lib.GemmDesc()
        d.a, d.b, d.c = 4096, 8192, 16384
        d.m, d.n, d.k, d.lda, d.ldb, d.ldc = 4, 4, 12, 12, 12, 4
        _lib.call('fvx_gemm', ctypes.byref(d), None)


def test_gemm_rejects_bad_row_groups():
    # a_row_group: 0 <= group <= stride < 2^31; grouped rows (m > group)
    # take a row-major bf16 A (no fragment-major A, no e4m3 A)
    lib = _lib.load()

    def desc(**kw):
        d = _lib.GemmDesc()
        d.a, d.b, d.c = 4096, 8192, 16384
        d.m, d.n, d.k, d.lda, d.ldb, d.ldc = 100, 64, 64, 64, 64, 64
        d.a_row_group, d.a_row_group_stride = 50, 51
        for k, v in kw.items():
            setattr(d, k, v)
        return d
    for kw in ({'a_row_group': -1}, {'a_row_group_stride': 49}, {'a_row_group_stride': 1 << 31}):
        assert lib.fvx_gemm(ctypes.byref(desc(**kw)), None) == _lib.FVX_ERR_SHAPE, kw
        assert 'a_row_group' in _err(lib), kw
    assert lib.fvx_gemm(ctypes.byref(desc(a_frag=1)), None) == _lib.FVX_ERR_ARG
    assert 'grouped A rows' in _err(lib)


def test_grouped_rows_views():
    # the Python layer reads a 3-D A with gaps between its groups as
    # grouped rows, and refuses other unevenly spaced views
    import torch

    from fluxvla_amd import kernels as K
    buf = torch.zeros(4, 51, 64)
    assert K._grouped_rows(buf[:, 1:]) == (50, 51)
    assert K._grouped_rows(buf[:, :]) is None
    assert K._grouped_rows(buf[:1, 1:]) is None
    with pytest.raises(ValueError):
        K._rows_ld(buf[:, 1:], 'x')
    assert K._rows_ld(buf[:1, 1:], 'x') == (50, 64)
    with pytest.raises(ValueError):
        K._grouped_rows(buf[:, 1:, :32].transpose(0, 1))
