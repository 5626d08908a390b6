"""Parity of the backward ops behind guidance RTC with use_vjp
(csrc/backward.hip) against float64 torch autograd of the forward op on
the same inputs (the CPU), each op at the action expert's shapes.

Bars: fp32 outputs within 1e-4 relative (max|out - ref| / max|ref|; the
kernels compute in fp32), bf16 outputs within 1e-2 (one bf16 rounding),
index/byte work (transposes) bit-exact.
"""
import pytest
import torch
import torch.nn.functional as F

from tests.conftest import announce

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 1e-2


def rel_err(out, ref):
    out = out.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return ((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def randn(shape, seed, std=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(dtype)


@pytest.fixture(scope='module')
def K():
    from fluxvla_amd import kernels
    kernels._lib.load()
    return kernels


def rms_ref(x, dy, scale=None, dres=None, eps=1e-6):
    """float64 autograd of y = x rsqrt(mean(x^2) + eps) (1 + scale)."""
    xd = x.double().cpu().requires_grad_(True)
    y = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps)
    if scale is not None:
        y = y * (1.0 + scale.double().cpu())
    (g,) = torch.autograd.grad(y, xd, dy.double().cpu())
    return g + (dres.double().cpu() if dres is not None else 0.0)


@pytest.mark.parametrize('cols', [1024, 2048, 32 * 8])
@pytest.mark.parametrize('with_scale', [False, True])
def test_rms_norm_backward(K, cuda, cols, with_scale):
    announce(f'rms_norm_backward cols={cols} scale={with_scale}')
    m = 51
    x = randn((m, cols), 1, std=2.0)
    dy = randn((m, cols), 2, dtype=torch.float32)
    dres = randn((m, cols), 3, dtype=torch.float32)
    scale = randn((cols,), 4, std=0.3) if with_scale else None
    gate = randn((cols,), 5, std=0.5)
    out = torch.empty(m, cols, dtype=torch.float32, device=cuda)
    outb = torch.empty(m, cols, dtype=torch.bfloat16, device=cuda)
    K.rms_norm_backward(x.to(cuda), dy.to(cuda), out=out, out_bf16=outb,
                        dres=dres.to(cuda),
                        scale=scale.to(cuda) if with_scale else None,
                        gate=gate.to(cuda), eps=1e-6)
    ref = rms_ref(x, dy, scale, dres)
    assert rel_err(out, ref) <= F32_TOL
    assert rel_err(outb, ref * gate.double()) <= BF16_TOL


def test_rms_norm_backward_row_groups(K, cuda):
    """Rows mapped through groups (the action rows behind each sample's
    state row): x / out rows (m / 50) * 51 + 1 + m % 50; rows outside the
    map stay untouched."""
    announce('rms_norm_backward row groups')
    B, Ss, na, cols = 3, 51, 50, 1024
    x = randn((B * Ss, cols), 11)
    dy = randn((B * na, cols), 12, dtype=torch.float32)
    out = torch.full((B * Ss, cols), 7.0, device=cuda)
    xg = x.to(cuda)
    # the view starting at row 1 of sample 0
    K.rms_norm_backward(xg[1:], dy.to(cuda), out=out[1:], row_group=na,
                        row_group_stride=Ss)
    xs = x.view(B, Ss, cols)[:, 1:].reshape(-1, cols)
    ref = rms_ref(xs, dy)
    got = out.view(B, Ss, cols)[:, 1:].reshape(-1, cols)
    assert rel_err(got, ref) <= F32_TOL
    assert (out.view(B, Ss, cols)[:, 0].cpu() == 7.0).all()


def test_geglu_backward(K, cuda):
    announce('act_backward geglu')
    m, n = 51, 4096
    gu = randn((m, 2 * n), 21, std=1.5)
    dh = randn((m, n), 22)
    out = K.act_backward(K._lib.ACT_BWD_GEGLU, gu.to(cuda), dh.to(cuda))
    g = gu[:, :n].double().requires_grad_(True)
    u = gu[:, n:].double().requires_grad_(True)
    h = F.gelu(g, approximate='tanh') * u
    dg, du = torch.autograd.grad(h, (g, u), dh.double())
    assert rel_err(out[:, :n], dg) <= BF16_TOL
    assert rel_err(out[:, n:], du) <= BF16_TOL


def test_silu_backward(K, cuda):
    announce('act_backward silu')
    m, n = 50, 1024
    z = randn((m, n), 31, std=3.0)
    dy = randn((m, n), 32)
    out = K.act_backward(K._lib.ACT_BWD_SILU, z.to(cuda), dy.to(cuda))
    zd = z.double().requires_grad_(True)
    (ref,) = torch.autograd.grad(F.silu(zd), zd, dy.double())
    assert rel_err(out, ref) <= BF16_TOL


def softmax_bwd_ref(s, dp, vis, scale):
    sd = s.double().cpu().requires_grad_(True)
    logits = (sd * scale).masked_fill(~vis, float('-inf'))
    p = torch.softmax(logits, -1).nan_to_num(0.0)
    (ds,) = torch.autograd.grad(p, sd, dp.double().cpu())
    return p.detach(), ds


@pytest.mark.parametrize('S', [816, 1100])
def test_attention_rows_backward(K, cuda, S):
    """The expert's suffix rows (51 tokens x 8 heads) over S prefix keys
    with padding and the block-causal suffix pattern; ds matches autograd of
    the masked softmax, ds_t / p_t hold the suffix columns transposed.  816:
    the row held in registers; 1100 (> 1024 keys): the multi-pass kernel."""
    announce(f'attention_rows_backward S={S}')
    Ss, H = 51, 8
    T = (S + Ss + 7) // 8 * 8
    nk = S + Ss
    rows = Ss * H
    scale = 256 ** -0.5
    s = randn((rows, T), 41, std=20.0, dtype=torch.float32)
    dp = randn((rows, T), 42, dtype=torch.float32)
    kgrp = torch.zeros(nk, dtype=torch.int32)
    kgrp[700:S] = 2**31 - 1  # padded prefix keys
    suf = torch.cumsum(torch.tensor([1, 1] + [0] * (Ss - 2)), 0).int()
    kgrp[S:] = suf
    qgrp = suf.clone()
    ds = torch.full((rows, T), float('nan'), dtype=torch.bfloat16, device=cuda)
    ds_t = torch.zeros(Ss, rows, dtype=torch.bfloat16, device=cuda)
    p_t = torch.zeros(Ss, rows, dtype=torch.bfloat16, device=cuda)
    K.attention_rows_backward(s.to(cuda), dp.to(cuda), ds, heads=H, n_keys=nk,
                              scale=scale, kgrp=kgrp.to(cuda),
                              qgrp=qgrp.to(cuda), ds_t=ds_t, p_t=p_t, key0=S,
                              n_suffix=Ss)
    tok = torch.arange(rows) // H
    vis = kgrp[None, :].long() <= qgrp[tok][:, None].long()
    p, ref = softmax_bwd_ref(s[:, :nk], dp[:, :nk], vis, scale)
    got = ds.cpu()
    assert torch.isfinite(got.float()).all()
    assert rel_err(got[:, :nk], ref) <= BF16_TOL
    assert (got[:, nk:].float() == 0).all()
    assert (got[:, :nk].float()[~vis] == 0).all()
    assert rel_err(ds_t.t(), ref[:, S:]) <= BF16_TOL
    assert rel_err(p_t.t(), p[:, S:]) <= BF16_TOL


@pytest.mark.parametrize('shape', [(3, 816, 256), (1, 51, 2048), (2, 37, 45)])
def test_transpose(K, cuda, shape):
    announce(f'transpose {shape}')
    src = randn(shape, 51).to(cuda)
    dst = torch.empty(shape[0], shape[2], shape[1], dtype=torch.bfloat16,
                      device=cuda)
    K.transpose(src, dst)
    assert torch.equal(dst.cpu(), src.cpu().transpose(1, 2))


def test_transpose_strided_views(K, cuda):
    """Cache slices: a [B, rows, D] slab of a longer cache into columns of
    a [B, D, T] one."""
    announce('transpose strided views')
    B, T, D, S, Ss = 2, 872, 256, 816, 51
    kc = randn((B, T, D), 52).to(cuda)
    kt = torch.zeros(B, D, T, dtype=torch.bfloat16, device=cuda)
    K.transpose(kc[:, S:S + Ss], kt[:, :, S:S + Ss])
    want = torch.zeros(B, D, T, dtype=torch.bfloat16)
    want[:, :, S:S + Ss] = kc.cpu()[:, S:S + Ss].transpose(1, 2)
    assert torch.equal(kt.cpu(), want)


def test_rope_backward(K, cuda):
    """Against float64 autograd of the forward rotation of pair (2i, 2i+1)
    by the fp32 table entry at the row's position."""
    announce('rope_backward')
    m, H, D = 51, 8, 256
    rope = K.rope_table(1024, D)
    pos = torch.randint(0, 1024, (m,), generator=torch.Generator().manual_seed(3),
                        dtype=torch.int32)
    dq = randn((m, H * D), 61, dtype=torch.float32)
    dk = randn((m, D), 62, dtype=torch.float32)
    dv = randn((m, D), 63, dtype=torch.float32)
    out = torch.empty(m, (H + 2) * D, dtype=torch.bfloat16, device=cuda)
    K.rope_backward(dq.to(cuda), dk.to(cuda), dv.to(cuda), rope.to(cuda),
                    pos.to(cuda), out, H, D)
    cs = rope[pos.long()].double()  # [m, D/2, 2]
    c, s = cs[..., 0], cs[..., 1]

    def fwd(x, heads):
        x = x.view(m, heads, D // 2, 2)
        a, b = x[..., 0], x[..., 1]
        return torch.stack([a * c[:, None] - b * s[:, None],
                            b * c[:, None] + a * s[:, None]], -1).reshape(m, -1)

    q = torch.zeros(m, H * D, dtype=torch.float64, requires_grad=True)
    k = torch.zeros(m, D, dtype=torch.float64, requires_grad=True)
    gq, gk = torch.autograd.grad((fwd(q, H), fwd(k, 1)), (q, k),
                                 (dq.double(), dk.double()))
    got = out.cpu()
    assert rel_err(got[:, :H * D], gq) <= BF16_TOL
    assert rel_err(got[:, H * D:(H + 1) * D], gk) <= BF16_TOL
    assert torch.equal(got[:, (H + 1) * D:], dv.to(torch.bfloat16))


def test_rtc_vjp_error_and_update(K, cuda):
    announce('rtc_vjp error / update')
    B, na, ad = 2, 50, 32
    x = randn((B * na, ad), 71, dtype=torch.float32)
    u = randn((B * na, ad), 72, dtype=torch.float32)
    prev = randn((B * na, ad), 73, dtype=torch.float32)
    g = randn((B * na, ad), 74, dtype=torch.float32)
    w = torch.rand(na, generator=torch.Generator().manual_seed(75))
    w[30:] = 0
    omt, dt, gw = 0.7, -0.1, 3.25
    e = torch.empty(B * na, ad, dtype=torch.bfloat16, device=cuda)
    K.rtc_vjp_error(x.to(cuda), u.to(cuda), prev.to(cuda), w.to(cuda), e, omt)
    wr = w.double().repeat(B)[:, None]
    ref_e = wr * (prev.double() - x.double() + omt * u.double())
    assert rel_err(e, ref_e) <= BF16_TOL
    xg = x.to(cuda)
    xb = torch.empty(B * na, ad, dtype=torch.bfloat16, device=cuda)
    gwt = torch.tensor([gw], dtype=torch.float32, device=cuda)
    K.rtc_vjp_update(xg, u.to(cuda), prev.to(cuda), w.to(cuda), g.to(cuda),
                     gwt, omt, dt, x_bf16=xb)
    ref = (x.double() + dt * u.double() - dt * gw * ref_e
           + dt * gw * omt * g.double())
    assert rel_err(xg, ref) <= F32_TOL
    assert torch.equal(xb.cpu(), xg.cpu().to(torch.bfloat16))


def test_attention_suffix_kv_backward(K, cuda):
    """dk = ds_t @ q and dv = p_t @ dO over the 408 query rows, against
    float64 products of the same bf16 operands."""
    announce('attention_suffix_kv_backward')
    Ss, R, D = 51, 408, 256
    ds_t = randn((Ss, R), 81, std=0.1)
    p_t = randn((Ss, R), 82, std=0.1)
    q = randn((R, D), 83)
    do = randn((R, D), 84)
    dk = torch.full((Ss, D), float('nan'), device=cuda)
    dv = torch.full((Ss, D), float('nan'), device=cuda)
    K.attention_suffix_kv_backward(ds_t.to(cuda), p_t.to(cuda), q.to(cuda),
                                   do.to(cuda), dk, dv)
    assert rel_err(dk, ds_t.double() @ q.double()) <= F32_TOL
    assert rel_err(dv, p_t.double() @ do.double()) <= F32_TOL


def test_geglu_rows(K, cuda):
    """out = gelu_tanh(gate) * up from stored [gate | up] rows, against
    float64 of the same bf16 inputs."""
    announce('geglu_rows')
    m, n = 51, 4096
    gu = randn((m, 2 * n), 91, std=1.5)
    out = K.geglu_rows(gu.to(cuda))
    g, u = gu[:, :n].double(), gu[:, n:].double()
    assert rel_err(out, F.gelu(g, approximate='tanh') * u) <= BF16_TOL


@pytest.mark.parametrize('n,S', [(1, 816), (2, 816), (1, 100)])
def test_attention_backward_fused(K, cuda, n, S):
    """The fused decode-shape attention backward (and the suffix keys'
    gradients from its ds_t / p_t) against float64 autograd of the masked
    attention: rows = 51 tokens x 8 heads, S prefix keys (some padded) plus
    the block-causal suffix; dq summed from the key-tile partials."""
    announce(f'attention_backward fused n={n} S={S}')
    Ss, H, D = 51, 8, 256
    nk, R = S + Ss, Ss * H
    T = (nk + 7) // 8 * 8
    scale = D ** -0.5
    q = randn((n, R, D), 101)
    k = randn((n, T, D), 102)
    v = randn((n, T, D), 103)
    dout = randn((n, R, D), 104)
    kgrp = torch.zeros(n, nk, dtype=torch.int32)
    kgrp[:, S - 30:S] = 2**31 - 1
    if n > 1:
        kgrp[1, :20] = 2**31 - 1
    suf = torch.cumsum(torch.tensor([1, 1] + [0] * (Ss - 2)), 0).int()
    kgrp[:, S:] = suf
    qgrp = suf[None].expand(n, Ss).contiguous()
    tok = torch.arange(R) // H
    vis = kgrp[:, None, :].long() <= qgrp[:, tok][:, :, None].long()  # [n, R, nk]
    qd = q.double().requires_grad_(True)
    kd = k[:, :nk].double().requires_grad_(True)
    vd = v[:, :nk].double().requires_grad_(True)
    logits = (qd @ kd.transpose(1, 2) * scale).masked_fill(~vis, float('-inf'))
    p = torch.softmax(logits, -1)
    o = p @ vd
    dq_ref, dk_ref, dv_ref = torch.autograd.grad(o, (qd, kd, vd), dout.double())
    # the copies the kernel reads hold the prefix keys only: the suffix
    # keys' kt columns and v rows come from the refresh (k, and vt = v^T)
    kt = torch.zeros(n, D, T, dtype=torch.bfloat16)
    kt[:, :, :S] = k[:, :S].transpose(1, 2)
    vrow = v.clone()
    vrow[:, S:] = 0
    vt = v.transpose(1, 2).contiguous()
    parts = K.attention_backward_parts(nk)
    dq = torch.full((parts, n * R, D), float('nan'), device=cuda)
    stats = torch.empty(2 * n * parts * R, device=cuda)
    ds_t = torch.zeros(n, Ss, R, dtype=torch.bfloat16, device=cuda)
    p_t = torch.zeros(n, Ss, R, dtype=torch.bfloat16, device=cuda)
    kc = k.to(cuda)
    vc, ktc = vrow.to(cuda), kt.to(cuda)
    K.attention_backward(q.to(cuda), o.detach().to(torch.bfloat16).to(cuda),
                         dout.to(cuda), kc[:, :nk], vc[:, :nk], ktc, dq,
                         stats, heads=H, scale=scale, kgrp=kgrp.to(cuda),
                         qgrp=qgrp.to(cuda), ds_t=ds_t, p_t=p_t, key0=S,
                         n_suffix=Ss, vt=vt.to(cuda), refresh=(S, Ss))
    want_kt = torch.zeros(n, D, T, dtype=torch.bfloat16)
    want_kt[:, :, :nk] = k[:, :nk].transpose(1, 2)
    assert torch.equal(ktc.cpu(), want_kt)
    assert torch.equal(vc.cpu()[:, :nk], v[:, :nk])
    got = dq.sum(0).view(n, R, D)
    assert torch.isfinite(got).all()
    assert rel_err(got, dq_ref) <= 2e-2
    # P and dS of the suffix keys
    ds_ref = p.detach() * (dout.double() @ vd.detach().transpose(1, 2)
                           - (o.detach() * dout.double()).sum(-1, keepdim=True)) * scale
    assert rel_err(p_t.transpose(1, 2), p.detach()[:, :, S:]) <= BF16_TOL
    assert rel_err(ds_t.transpose(1, 2), ds_ref[:, :, S:]) <= 2e-2
    for z in range(n):
        dk = torch.empty(Ss, D, device=cuda)
        dv = torch.empty(Ss, D, device=cuda)
        K.attention_suffix_kv_backward(ds_t[z], p_t[z], q[z].to(cuda),
                                       dout[z].to(cuda), dk, dv)
        assert rel_err(dk, dk_ref[z, S:]) <= 2e-2
        assert rel_err(dv, dv_ref[z, S:]) <= 2e-2


def test_fragment_major_outputs(K, cuda):
    """The fragment-major copies (the A operands of the bs=1 backward GEMMs)
    hold exactly the row-major outputs' values, laid out as FragA."""
    announce('backward fragment-major outputs')
    m, hid, mlp, H, D = 51, 1024, 4096, 8, 256
    x = randn((m, hid), 111).to(cuda)
    dy = randn((m, hid), 112, dtype=torch.float32).to(cuda)
    gate = randn((hid,), 113).to(cuda)
    outb = torch.empty(m, hid, dtype=torch.bfloat16, device=cuda)
    fa = K.FragA.empty(hid, cuda).rows(m)
    K.rms_norm_backward(x, dy, out_bf16=outb, out_frag=fa, gate=gate)
    assert torch.equal(fa.buf, K.pack_frag_a_ref(outb))
    gu = randn((m, 2 * mlp), 114).to(cuda)
    dh = randn((m, mlp), 115).to(cuda)
    row = K.act_backward(K._lib.ACT_BWD_GEGLU, gu, dh)
    fg = K.FragA.empty(2 * mlp, cuda).rows(m)
    K.act_backward(K._lib.ACT_BWD_GEGLU, gu, dh, out_frag=fg)
    assert torch.equal(fg.buf, K.pack_frag_a_ref(row))
    h = K.geglu_rows(gu)
    fh = K.FragA.empty(mlp, cuda).rows(m)
    K.geglu_rows(gu, out_frag=fh)
    assert torch.equal(fh.buf, K.pack_frag_a_ref(h))
    rope = K.rope_table(1024, D).to(cuda)
    pos = torch.arange(m, dtype=torch.int32, device=cuda) * 7
    dq = randn((m, H * D), 116, dtype=torch.float32).to(cuda)
    dk = randn((m, D), 117, dtype=torch.float32).to(cuda)
    dv = randn((m, D), 118, dtype=torch.float32).to(cuda)
    out = torch.empty(m, (H + 2) * D, dtype=torch.bfloat16, device=cuda)
    K.rope_backward(dq, dk, dv, rope, pos, out, H, D)
    fq = K.FragA.empty((H + 2) * D, cuda).rows(m)
    K.rope_backward(dq, dk, dv, rope, pos, None, H, D, out_frag=fq)
    assert torch.equal(fq.buf, K.pack_frag_a_ref(out))


@pytest.mark.parametrize('m', [51, 102])
def test_geglu_gemm_keeps_pre_activations(K, cuda, m):
    """fvx_gemm_desc.gu_out: the GeGLU GEMM (skinny at M = 51, tiled at
    102; rownorm) also stores the gate and up values its product is taken
    from -- against float64, and its product bitwise the same as without."""
    announce(f'geglu gu_out m={m}')
    k, n = 1024, 4096
    a = randn((m, k), 121, std=2.0).to(cuda)
    wg = randn((n, k), 122, std=0.03).to(cuda)
    wu = randn((n, k), 123, std=0.03).to(cuda)
    gu = torch.full((m, 2 * n), float('nan'), dtype=torch.bfloat16, device=cuda)
    h = K.gemm_geglu(a, wg, wu, rownorm_eps=1e-6, gu_out=gu)
    h0 = K.gemm_geglu(a, wg, wu, rownorm_eps=1e-6)
    assert torch.equal(h, h0)
    ad = a.double().cpu()
    xn = ad * torch.rsqrt(ad.pow(2).mean(-1, keepdim=True) + 1e-6)
    assert rel_err(gu[:, :n], xn @ wg.double().cpu().t()) <= BF16_TOL
    assert rel_err(gu[:, n:], xn @ wu.double().cpu().t()) <= BF16_TOL


@pytest.mark.parametrize('groups', [1, 2])
def test_qkv_rope_writes_backward_copies(K, cuda, groups):
    """fvx_gemm_desc.k_t_out / v_rows_out: the QKV + RoPE GEMM with a
    transposed value cache also writes the keys transposed and the values
    row-major (the attention backward's operands) -- bitwise the transposes
    of what it writes to k_out / v_out, at the cache's row groups and gaps,
    and nothing outside the suffix columns / rows."""
    announce(f'qkv_rope backward copies groups={groups}')
    ss, pre, hd, nq, k = 51, 816, 256, 8, 1024
    T, m = pre + ss, groups * ss
    a = randn((m, k), 131, std=2.0).to(cuda)
    w = randn(((nq + 2) * hd, k), 132, std=0.03).to(cuda)
    pos = torch.arange(pre, pre + ss, dtype=torch.int32).repeat(groups).to(cuda)
    rope = K.rope_table(T + 8, hd, device=cuda)
    q = torch.empty(m, nq * hd, dtype=torch.bfloat16, device=cuda)
    kc = torch.zeros(groups, T, hd, dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros(groups, hd, T, dtype=torch.bfloat16, device=cuda)
    kt = torch.zeros(groups, hd, T, dtype=torch.bfloat16, device=cuda)
    vr = torch.zeros(groups, T, hd, dtype=torch.bfloat16, device=cuda)
    K.gemm_qkv_rope(a, w, rope, pos, q, kc.view(groups * T, hd)[pre:],
                    vc[:, :, pre:], nq, hd, rownorm_eps=1e-6, row_group=ss,
                    row_group_stride=T, v_ld=T, k_t_out=kt[:, :, pre:], kt_ld=T,
                    v_rows_out=vr.view(groups * T, hd)[pre:])
    assert torch.equal(kt, kc.transpose(1, 2))
    assert torch.equal(vr, vc.transpose(1, 2))
    assert kc[:, pre:].abs().max().item() > 0
    assert kc[:, :pre].abs().max().item() == 0.0
    assert vc[:, :, :pre].abs().max().item() == 0.0
