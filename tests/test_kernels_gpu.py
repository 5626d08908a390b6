"""Parity of every HIP kernel against an fp32 reference of the same op.

References are computed on the CPU in fp32 (float64 where noted) from the
same bf16 inputs the kernel sees.  Bar (from the north star): each bf16 op
has max relative error <= 1e-2, measured as max|out - ref| / max|ref|.
"""
import pytest
import torch
import torch.nn.functional as F

from tests.conftest import announce

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2


def rel_err(out, ref):
    out = out.detach().float().cpu()
    ref = ref.detach().float().cpu()
    return ((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(shape, seed, std=1.0, mean=0.0):
    return (torch.randn(shape, generator=gen(seed)) * std + mean).to(
        torch.bfloat16)


@pytest.fixture(scope='module')
def K():
    from fluxvla_amd import kernels
    kernels._lib.load()
    return kernels


# ---------------------------------------------------------------------------
# Norms
# ---------------------------------------------------------------------------
def test_rms_norm_residual_config1(K, cuda):
    """Config 1: x, residual [1024, 2048] ~N(0,1), w ~N(1, 0.02), eps 1e-6."""
    announce('rms_norm_residual [1024,2048]')
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1024, 2048, generator=g).bfloat16()
    res = torch.randn(1024, 2048, generator=g).bfloat16()
    w = (torch.randn(2048, generator=g) * 0.02 + 1.0).bfloat16()
    y, r = K.rms_norm_residual(x.to(cuda), res.to(cuda), w.to(cuda), 1e-6,
                               residual_out=torch.empty_like(x, device=cuda))
    h = x.float() + res.float()
    ref_y = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    assert rel_err(y, ref_y) <= REL_TOL
    assert rel_err(r, h) <= REL_TOL
    # residual_out is exactly bf16(x + res) (one rounding of an exact sum)
    assert torch.equal(r.cpu(), h.bfloat16())


@pytest.mark.parametrize('rows,cols', [(51, 1024), (816, 2048), (7, 1152)])
def test_rms_norm_plain(K, cuda, rows, cols):
    announce(f'rms_norm plain [{rows},{cols}]')
    x = randn((rows, cols), 1)
    y, _ = K.rms_norm_residual(x.to(cuda), None, None, 1e-6)
    xf = x.float()
    ref = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    assert rel_err(y, ref) <= REL_TOL


def test_layer_norm(K, cuda):
    announce('layer_norm [768,1152]')
    x = randn((768, 1152), 2, std=3.0, mean=0.5)
    w = randn((1152,), 3, std=0.1, mean=1.0)
    b = randn((1152,), 4, std=0.1)
    y = K.layer_norm(x.to(cuda), w.to(cuda), b.to(cuda), 1e-6)
    ref = F.layer_norm(x.float(), (1152,), w.float(), b.float(), 1e-6)
    assert rel_err(y, ref) <= REL_TOL


def test_adarms_norm(K, cuda):
    announce('adarms_norm [100,1024] 2 styles')
    x = randn((100, 1024), 5)
    style = randn((2, 3072), 6, std=0.2)
    y = torch.empty(100, 1024, dtype=torch.bfloat16, device=cuda)
    gt = torch.empty_like(y)
    K.adarms_norm(x.to(cuda), style.to(cuda), y, gt, rows_per_style=50)
    xf = x.float()
    n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    st = style.float().repeat_interleave(50, 0)
    ref = n * (1 + st[:, :1024]) + st[:, 1024:2048]
    assert rel_err(y, ref) <= REL_TOL
    assert torch.equal(gt.cpu(), style[:, 2048:].repeat_interleave(50, 0))


# ---------------------------------------------------------------------------
# GEMM family
# ---------------------------------------------------------------------------
GEMM_SHAPES = [
    # (M, N, K): skinny (M <= 64) and tiled, ragged edges included
    (51, 2560, 1024), (50, 1024, 32), (1, 1024, 1024), (64, 4304, 1152),
    (816, 2560, 2048), (768, 4304, 1152), (768, 1152, 4304), (200, 640, 96),
    (129, 136, 72),
]


@pytest.mark.parametrize('m,n,k', GEMM_SHAPES)
def test_gemm_plain_bias_act(K, cuda, m, n, k):
    announce(f'gemm plain m={m} n={n} k={k}')
    a = randn((m, k), 10)
    w = randn((n, k), 11, std=0.02)
    b = randn((n,), 12, std=0.5)
    ref = a.float() @ w.float().t()
    out = K.gemm(a.to(cuda), w.to(cuda))
    assert rel_err(out, ref) <= REL_TOL
    out = K.gemm(a.to(cuda), w.to(cuda), bias=b.to(cuda), act=2)
    assert rel_err(out, F.gelu(ref + b.float(), approximate='tanh')) <= REL_TOL
    out = K.gemm(a.to(cuda), w.to(cuda), bias=b.to(cuda), act=1)
    assert rel_err(out, F.silu(ref + b.float())) <= REL_TOL


@pytest.mark.parametrize('m', [51, 816])
def test_gemm_residual_gate_inplace(K, cuda, m):
    announce(f'gemm residual/gate in place m={m}')
    n, k = 1024, 2048
    a = randn((m, k), 20)
    w = randn((n, k), 21, std=0.02)
    res = randn((m, n), 22)
    gate = randn((m, n), 23, std=0.5)
    ref = a.float() @ w.float().t()
    x = res.clone().to(cuda)
    K.gemm(a.to(cuda), w.to(cuda), out=x, residual=x)
    assert rel_err(x, res.float() + ref) <= REL_TOL
    x = res.clone().to(cuda)
    K.gemm(a.to(cuda), w.to(cuda), out=x, residual=x, gate=gate.to(cuda))
    assert rel_err(x, res.float() + ref * gate.float()) <= REL_TOL


def test_gemm_split_deterministic(K, cuda):
    """Split-K partials are reduced in a fixed order: bitwise repeatable,
    and equal (to rounding) to the single-pass kernel."""
    announce('gemm split-k determinism')
    a = randn((51, 4096), 30).to(cuda)
    w = randn((1024, 4096), 31, std=0.02).to(cuda)
    o1 = K.gemm(a, w)
    o2 = K.gemm(a, w)
    o3 = K.gemm(a, w, split_k=1)
    assert torch.equal(o1, o2)
    assert rel_err(o1, o3.float()) <= 4e-3


@pytest.mark.parametrize('m,n,k', [(51, 1000, 1000), (7, 1004, 744),
                                   (64, 72, 4096), (33, 520, 264)])
def test_gemm_skinny_ragged(K, cuda, m, n, k):
    """M <= 64: partial column tiles, a partial last K range, N % 8 != 0 (the
    element-wise epilogue) and an output row stride that is not a multiple
    of 8 (element-wise stores everywhere), with bias + residual in place."""
    announce(f'gemm skinny ragged m={m} n={n} k={k}')
    a = randn((m, k), 24)
    w = randn((n, k), 25, std=0.02)
    b = randn((n,), 26, std=0.5)
    res = randn((m, n), 27)
    ref = a.float() @ w.float().t() + b.float() + res.float()
    x = res.clone().to(cuda)
    K.gemm(a.to(cuda), w.to(cuda), out=x, bias=b.to(cuda), residual=x)
    assert rel_err(x, ref) <= REL_TOL
    wide = torch.zeros(m, n + 3, dtype=torch.bfloat16, device=cuda)
    wide[:, :n] = res.to(cuda)
    K.gemm(a.to(cuda), w.to(cuda), out=wide[:, :n], bias=b.to(cuda),
           residual=wide[:, :n])
    assert rel_err(wide[:, :n], ref) <= REL_TOL
    assert wide[:, n:].abs().max().item() == 0.0


def test_gemm_split_counters_left_zero(K, cuda):
    """The split-K arrival counters (first 4 KiB of the GEMM workspace) are
    zero after every call, so back-to-back calls of different shapes and
    modes each see a clean start; repeated calls are bitwise equal."""
    announce('gemm split counters')
    ws = K.workspace(cuda)
    a = randn((51, 2048), 28).to(cuda)
    w1 = randn((1024, 2048), 29, std=0.02).to(cuda)
    w2 = randn((4096, 2048), 31, std=0.02).to(cuda)
    outs = []
    for _ in range(3):
        outs.append(K.gemm(a, w1))
        K.gemm_geglu(a, w2, w1.repeat(4, 1).contiguous(), rownorm_eps=1e-6)
        assert ws[:4096].count_nonzero().item() == 0
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


@pytest.mark.parametrize('m,n,k', [(51, 2560, 1024), (51, 1024, 4096),
                                   (50, 32, 1024), (17, 1024, 32)])
def test_gemm_fragment_major_operands(K, cuda, m, n, k):
    """FragA / FragB operands feed the MFMAs the same fragments in the same
    k order as row-major ones: the outputs are bitwise equal.  c_frag holds
    the output in the FragA layout (rows < m)."""
    announce(f'gemm fragment-major m={m} n={n} k={k}')
    a = randn((m, k), 32).to(cuda)
    w = randn((n, k), 33, std=0.02).to(cuda)
    b = randn((n,), 34, std=0.5).to(cuda)
    res = randn((m, n), 35).to(cuda)
    af = K.FragA.empty(k, cuda).rows(m)
    K.pack_frag(a, af)
    ref_pack = K.pack_frag_a_ref(a.cpu())
    mask = K.pack_frag_a_ref(torch.ones(m, k, dtype=torch.bfloat16)) != 0
    assert torch.equal(af.buf.cpu()[mask], ref_pack[mask])
    wf = K.FragB.pack(w)
    x0 = res.clone()
    K.gemm(a, w, out=x0, bias=b, residual=x0)
    for aa, ww in ((af, w), (a, wf), (af, wf)):
        x1 = res.clone()
        cf = K.FragA.empty(n, cuda).rows(m) if n % 32 == 0 else None
        K.gemm(aa, ww, out=x1, bias=b, residual=x1, c_frag=cf)
        assert torch.equal(x0, x1)
        if cf is not None:
            assert torch.equal(cf.buf.cpu()[K.pack_frag_a_ref(
                torch.ones(m, n, dtype=torch.bfloat16)) != 0],
                K.pack_frag_a_ref(x1.cpu())[K.pack_frag_a_ref(
                    torch.ones(m, n, dtype=torch.bfloat16)) != 0])
    if n % 16 == 0 and k >= 256:
        g0 = K.gemm_geglu(a, w, w.flip(0).contiguous(), rownorm_eps=1e-6)
        g1 = K.gemm_geglu(af, wf, K.FragB.pack(w.flip(0).contiguous()),
                          rownorm_eps=1e-6)
        assert torch.equal(g0, g1)


@pytest.mark.parametrize('m', [40, 96])
def test_bf16_rounding_matches_torch(K, cuda, m):
    """The kernels' fp32 -> bf16 conversion rounds to nearest even, as
    torch's cast does: the bf16 output of a GEMM equals torch's cast of the
    same GEMM's fp32 output bit for bit (outputs span ~12 binades)."""
    announce(f'bf16 rounding m={m}')
    a = randn((m, 256), 36, std=4.0).to(cuda)
    scale = torch.logspace(-6, 6, 512, base=2.0).bfloat16()[:, None]
    w = (randn((512, 256), 37) * scale).bfloat16().to(cuda)
    o32 = K.gemm(a, w, out_f32=True)
    o16 = K.gemm(a, w)
    assert torch.equal(o16.cpu(), o32.cpu().bfloat16())


def test_gemm_pos_rowgroup_f32(K, cuda):
    announce('gemm pos/row_group/out_f32')
    m, n, k = 768, 1152, 640
    a = randn((m, k), 40)
    w = randn((n, k), 41, std=0.02)
    b = randn((n,), 42)
    pos = randn((256, n), 43)
    ref = a.float() @ w.float().t() + b.float() + pos.float().repeat(3, 1)
    out = K.gemm(a.to(cuda), w.to(cuda), bias=b.to(cuda), pos=pos.to(cuda),
                 pos_period=256)
    assert rel_err(out, ref) <= REL_TOL
    # row remap: rows [256 g + r] -> [300 g + r] of a taller buffer
    big = torch.zeros(900, n, dtype=torch.float32, device=cuda)
    K.gemm(a.to(cuda), w.to(cuda), out=big, bias=b.to(cuda), pos=pos.to(cuda),
           pos_period=256, out_f32=True, row_group=256, row_group_stride=300)
    got = big.view(3, 300, n)[:, :256].reshape(768, n)
    assert rel_err(got, ref) <= REL_TOL
    assert big.view(3, 300, n)[:, 256:].abs().max().item() == 0.0


@pytest.mark.parametrize('m,n,act,rg', [
    (768, 3456, 'none', 0),      # SigLIP Q|K|V (64 x 128 tiles)
    (1024, 4304, 'gelu', 0),     # fc1, tanh GELU
    (130, 1152, 'none', 0),      # ragged rows, 64 x 64 tiles
    (768, 2048, 'none', 256),    # projector: rows [256 g + r] -> [300 g + r]
])
def test_gemm_layernorm_fold(K, cuda, m, n, act, rg):
    """LayerNorm folded into the following GEMM: the GEMM sums its A rows'
    values and squares in the K loop and computes LayerNorm(x) @ W^T + b
    with W scaled by the norm's gain, the weight's column sums and the
    shift folded into an fp32 bias.  x has a mean offset (0.3) so the mean
    term matters.  Reference: torch fp32 layer_norm of the same bf16 x, then
    the fp32 GEMM with the unfolded weight (and tanh GELU)."""
    announce(f'gemm layernorm fold m={m} n={n} act={act} row_group={rg}')
    from fluxvla_amd._lib import ACT_GELU_TANH, ACT_NONE
    h = 1152
    x = randn((m, h), 62, mean=0.3)
    g = randn((h,), 63, std=0.2, mean=1.0)
    beta = randn((h,), 64, std=0.2)
    w = randn((n, h), 65, std=0.03)
    b = randn((n,), 66, std=0.2)
    wf = (w.float() * g.float()).bfloat16()
    csum = wf.float().sum(1)
    bf = b.float() + w.float() @ beta.float()
    ref = F.layer_norm(x.float(), (h,), g.float(), beta.float(), eps=1e-6) @ w.float().t() + b.float()
    if act == 'gelu':
        ref = F.gelu(ref, approximate='tanh')
    kw = dict(rownorm_eps=1e-6, ln_csum=csum.to(cuda), bias_f32=bf.to(cuda),
              act=ACT_GELU_TANH if act == 'gelu' else ACT_NONE)
    xc = x.to(cuda)
    if rg:
        groups = m // rg
        big = torch.zeros(groups * 300, n, dtype=torch.bfloat16, device=cuda)
        K.gemm(xc, wf.to(cuda), out=big, row_group=rg, row_group_stride=300, **kw)
        got = big.view(groups, 300, n)[:, :rg].reshape(m, n)
        assert big.view(groups, 300, n)[:, rg:].abs().max().item() == 0.0
    else:
        got = K.gemm(xc, wf.to(cuda), **kw)
    assert rel_err(got, ref) <= REL_TOL
    # repeatable bit for bit (fixed summation order)
    if not rg:
        assert torch.equal(got, K.gemm(xc, wf.to(cuda), **kw))


@pytest.mark.parametrize('m,n,k', [(51, 4096, 1024), (816, 16384, 2048),
                                   (100, 4096, 1024)])
def test_gemm_geglu_rownorm(K, cuda, m, n, k):
    announce(f'gemm geglu rownorm m={m} n={n} k={k}')
    x = randn((m, k), 50, std=2.0)
    wg = randn((n, k), 51, std=0.02)
    wu = randn((n, k), 52, std=0.02)
    out = K.gemm_geglu(x.to(cuda), wg.to(cuda), wu.to(cuda), rownorm_eps=1e-6)
    xf = x.float()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = F.gelu(xn @ wg.float().t(), approximate='tanh') * (xn @ wu.float().t())
    assert rel_err(out, ref) <= REL_TOL


def rope_ref(x, pos, hd, theta=10000.0):
    """Rotate-half RoPE on [rows, heads, hd] at integer positions (fp64)."""
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float64) / hd))
    ph = pos.double()[:, None] * inv[None, :]
    cos = torch.cat([ph.cos(), ph.cos()], -1)[:, None, :]
    sin = torch.cat([ph.sin(), ph.sin()], -1)[:, None, :]
    x1, x2 = x[..., :hd // 2], x[..., hd // 2:]
    rot = torch.cat([-x2, x1], -1)
    return x * cos + rot * sin


def interleave_perm(hd):
    """Row permutation that puts rotate-half pair (i, i + hd/2) at (2i, 2i+1)
    (condition_gemma_inference.py:46-63)."""
    idx = torch.arange(hd).view(2, hd // 2).t().reshape(-1)
    return idx


@pytest.mark.parametrize('m,k,start', [(51, 1024, 816), (816, 2048, 0),
                                         (102, 1024, 816)])
@pytest.mark.parametrize('vt', [False, True])
def test_gemm_qkv_rope(K, cuda, m, k, start, vt):
    announce(f'gemm qkv_rope m={m} k={k} v_transposed={vt}')
    nq, hd = 8, 256
    x = randn((m, k), 60, std=1.5)
    wq = randn((nq * hd, k), 61, std=0.02)
    wk = randn((hd, k), 62, std=0.02)
    wv = randn((hd, k), 63, std=0.02)
    perm = interleave_perm(hd)
    wq_p = wq.view(nq, hd, k)[:, perm].reshape(nq * hd, k)
    wk_p = wk[perm]
    w = torch.cat([wq_p, wk_p, wv], 0).contiguous()
    pos = torch.arange(start, start + m, dtype=torch.int32)
    rope = K.rope_table(start + m + 8, hd, device=cuda)
    q = torch.empty(m, nq * hd, dtype=torch.bfloat16, device=cuda)
    kk = torch.zeros(m + 10, hd, dtype=torch.bfloat16, device=cuda)
    vv = torch.zeros(m + 10, hd, dtype=torch.bfloat16, device=cuda)
    vtc = torch.zeros(hd, m + 24, dtype=torch.bfloat16, device=cuda)
    K.gemm_qkv_rope(x.to(cuda), w.to(cuda), rope, pos.to(cuda), q, kk[5:],
                    vtc[:, 8:] if vt else vv[5:], nq, hd, rownorm_eps=1e-6,
                    v_ld=m + 24 if vt else None)
    if vt:
        assert vtc[:, :8].abs().max().item() == 0.0
        vv[5:5 + m] = vtc[:, 8:8 + m].t()
    xf = x.double()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    rq = rope_ref((xn @ wq.double().t()).view(m, nq, hd), pos, hd)
    rk = rope_ref((xn @ wk.double().t()).view(m, 1, hd), pos, hd)
    rv = xn @ wv.double().t()
    got_q = q.cpu().view(m, nq, hd)[:, :, torch.argsort(perm)]
    got_k = kk[5:5 + m].cpu()[:, torch.argsort(perm)]
    assert rel_err(got_q, rq) <= REL_TOL
    assert rel_err(got_k, rk.view(m, hd)) <= REL_TOL
    assert rel_err(vv[5:5 + m], rv) <= REL_TOL
    assert kk[:5].abs().max().item() == 0.0
    assert kk[5 + m:].abs().max().item() == 0.0


@pytest.mark.parametrize('m', [50, 400])
def test_gemm_euler(K, cuda, m):
    announce(f'gemm euler m={m}')
    x = randn((m, 1024), 70, std=2.0)
    w = randn((32, 1024), 71, std=0.02)
    b = randn((32,), 72, std=0.1)
    xt0 = torch.randn(m, 32, generator=gen(73))
    xt = xt0.clone().to(cuda)
    xtb = torch.empty(m, 32, dtype=torch.bfloat16, device=cuda)
    K.gemm_euler(x.to(cuda), w.to(cuda), b.to(cuda), xt, -0.1, xt_bf16=xtb,
                 rownorm_eps=1e-6)
    xf = x.float()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    v = xn @ w.float().t() + b.float()
    ref = xt0 - 0.1 * v
    assert (xt.cpu() - ref).abs().max().item() <= 2e-3
    assert torch.equal(xtb.cpu(), xt.cpu().bfloat16())


@pytest.mark.parametrize('groups,rows,stride', [(8, 50, 51), (2, 25, 51), (3, 50, 64),
                                                (32, 50, 51)])
def test_gemm_grouped_a_rows(K, cuda, groups, rows, stride):
    """A read in row groups with gaps between them (the action rows behind
    each sample's state row: fvx_gemm_desc.a_row_group), as a 3-D view
    [groups, rows, k] of a taller buffer.  The Euler GEMM over the batch
    against the same GEMM on the gathered rows, bit for bit (same
    products, same tile order), and against an fp32 reference; a PLAIN
    GEMM with bias on the same view; the gap rows are never read (NaN)."""
    announce(f'gemm grouped A rows {groups}x{rows} stride {stride}')
    k, n = 1024, 32
    buf = randn((groups, stride, k), 74, std=2.0)
    buf[:, :stride - rows] = float('nan')
    xg = buf.to(cuda)[:, stride - rows:]
    x = xg.contiguous()
    w = randn((n, k), 75, std=0.02).to(cuda)
    b = randn((n,), 76, std=0.1).to(cuda)
    m = groups * rows
    xt0 = torch.randn(m, n, generator=gen(77))
    outs = []
    for a in (xg, x):
        xt = xt0.clone().to(cuda)
        xtb = torch.empty(m, n, dtype=torch.bfloat16, device=cuda)
        K.gemm_euler(a, w, b, xt, -0.1, xt_bf16=xtb, rownorm_eps=1e-6)
        outs.append((xt.cpu(), xtb.cpu()))
    if m > 64:  # both take the tile kernel (m <= 64 ungrouped: the skinny one)
        assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    xf = x.view(m, k).float().cpu()
    v = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)) @ w.float().cpu().t() \
        + b.float().cpu()
    assert (outs[0][0] - (xt0 - 0.1 * v)).abs().max().item() <= 2e-3
    got = K.gemm(xg, w, bias=b)
    assert got.shape == (groups, rows, n)
    if m > 64:
        assert torch.equal(got, K.gemm(x, w, bias=b))
    assert rel_err(got.view(m, n), xf @ w.float().cpu().t() + b.float().cpu()) <= REL_TOL


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
def sdpa_ref(q, k, v, mask=None, scale=None):
    """q [B, H, Sq, D], k/v [B, 1, Sk, D] fp32 on CPU; mask [B, Sq, Sk]."""
    k = k.expand(-1, q.shape[1], -1, -1)
    v = v.expand(-1, q.shape[1], -1, -1)
    am = None if mask is None else mask[:, None]
    return F.scaled_dot_product_attention(q, k, v, attn_mask=am, scale=scale)


@pytest.mark.parametrize('splits', [0, 1])
@pytest.mark.parametrize('vt', [False, True])
def test_attention_prefix_mqa(K, cuda, splits, vt):
    announce(f'attention prefix mqa 816 splits={splits} v_transposed={vt}')
    S, H, D = 816, 8, 256
    q = randn((1, S, H, D), 80)
    k = randn((1, S, D), 81)
    v = randn((1, S, D), 82)
    o = torch.empty(1, S, H, D, dtype=torch.bfloat16, device=cuda)
    if vt:  # value cache [B, D, T] with spare token columns
        vv = torch.zeros(1, D, S + 56, dtype=torch.bfloat16)
        vv[:, :, :S] = v.transpose(1, 2)
        K.mqa_attention(q.to(cuda), k.to(cuda), vv.to(cuda), o,
                        kv_splits=splits, v_transposed=True)
    else:
        K.mqa_attention(q.to(cuda), k.to(cuda), v.to(cuda), o,
                        kv_splits=splits)
    ref = sdpa_ref(q.float().transpose(1, 2), k.float()[:, None],
                   v.float()[:, None]).transpose(1, 2)
    assert rel_err(o, ref) <= REL_TOL


def test_attention_prefix_padded(K, cuda):
    """Padded keys (pad mask) are invisible: kgrp = INT32_MAX there."""
    announce('attention prefix padded')
    S, H, D = 300, 8, 256
    pad = torch.ones(S, dtype=torch.bool)
    pad[200:256] = False  # a missing camera block in the middle
    pad[290:] = False     # prompt padding
    q = randn((1, S, H, D), 83)
    k = randn((1, S, D), 84)
    v = randn((1, S, D), 85)
    kgrp = torch.where(pad, 0, 2**31 - 1).to(torch.int32)[None]
    qgrp = torch.zeros(1, S, dtype=torch.int32)
    o = torch.empty(1, S, H, D, dtype=torch.bfloat16, device=cuda)
    K.mqa_attention(q.to(cuda), k.to(cuda), v.to(cuda), o, kgrp.to(cuda),
                    qgrp.to(cuda))
    mask = pad[None, None, :].expand(1, S, S)
    ref = sdpa_ref(q.float().transpose(1, 2), k.float()[:, None],
                   v.float()[:, None], mask).transpose(1, 2)
    assert rel_err(o[:, pad], ref[:, pad]) <= REL_TOL


@pytest.mark.parametrize('splits', [1, 2, 3])
@pytest.mark.parametrize('batch', [1, 2])
def test_attention_prefix_key_ranges(K, cuda, splits, batch):
    """Transposed value cache with ranges of >= 4 key tiles (the prefix
    kernel): 600 tokens x 8 heads are 75 row groups of 64, an odd count,
    so the last workgroup of a 128-row kernel has one group past the end;
    the last range is partial, and padded keys sit inside a range."""
    announce(f'attention prefix key ranges splits={splits} batch={batch}')
    S, H, D, T = 600, 8, 256, 640
    q = randn((batch, S, H, D), 86)
    k = randn((batch, T, D), 87)
    v = randn((batch, T, D), 88)
    kgrp = torch.zeros(batch, S, dtype=torch.int32)
    kgrp[-1, 130:170] = 2**31 - 1
    kgrp[:, 580:] = 2**31 - 1
    qgrp = torch.zeros(batch, S, dtype=torch.int32)
    o = torch.empty(batch, S, H, D, dtype=torch.bfloat16, device=cuda)
    vt = v.transpose(1, 2).contiguous().to(cuda)
    K.mqa_attention(q.to(cuda), k.to(cuda)[:, :S], vt, o, kgrp.to(cuda),
                    qgrp.to(cuda), kv_splits=splits, v_transposed=True)
    mask = (kgrp[:, None, :] <= qgrp[:, :, None])
    ref = sdpa_ref(q.float().transpose(1, 2), k[:, :S].float()[:, None],
                   v[:, :S].float()[:, None], mask).transpose(1, 2)
    assert rel_err(o, ref) <= REL_TOL


@pytest.mark.parametrize('splits', [0, 1, 5, 14])
@pytest.mark.parametrize('vt', [False, True])
@pytest.mark.parametrize('batch', [1, 3])
def test_attention_decode_block_causal(K, cuda, splits, vt, batch):
    """PI0 suffix: state token sees prefix + itself, actions see all.  With a
    transposed value cache this runs the LDS-tiled decode kernel (and, at
    batch 1, also writes the fragment-major copy of the output)."""
    announce(f'attention decode block-causal splits={splits} vt={vt} '
             f'batch={batch}')
    P, Ssuf, H, D = 816, 51, 8, 256
    T = P + Ssuf
    Ta = T + 13 if not vt else 872
    q = randn((batch, Ssuf, H, D), 90)
    cache_k = randn((batch, Ta, D), 91)
    cache_v = randn((batch, Ta, D), 92)
    att = torch.tensor([1, 1] + [0] * 49)
    cum = torch.cumsum(att, 0).to(torch.int32)
    kgrp = torch.cat([torch.zeros(P, dtype=torch.int32), cum])[None].repeat(
        batch, 1)
    kgrp[-1, 100:140] = 2**31 - 1  # padded prefix keys in the last sample
    qgrp = cum[None].repeat(batch, 1)
    o = torch.empty(batch, Ssuf, H, D, dtype=torch.bfloat16, device=cuda)
    kc = cache_k.to(cuda)
    if vt:
        vc = cache_v.transpose(1, 2).contiguous().to(cuda)
    else:
        vc = cache_v.to(cuda)[:, :T]
    of = K.FragA.empty(H * D, cuda).rows(Ssuf) if vt and batch == 1 else None
    K.mqa_attention(q.to(cuda), kc[:, :T], vc, o, kgrp.to(cuda),
                    qgrp.to(cuda), kv_splits=splits, v_transposed=vt,
                    o_frag=of)
    mask = (kgrp[:, None, :] <= qgrp[:, :, None])
    ref = sdpa_ref(q.float().transpose(1, 2), cache_k[:, :T].float()[:, None],
                   cache_v[:, :T].float()[:, None], mask).transpose(1, 2)
    assert rel_err(o, ref) <= REL_TOL
    if of is not None:
        valid = K.pack_frag_a_ref(torch.ones(Ssuf, H * D,
                                             dtype=torch.bfloat16)) != 0
        assert torch.equal(of.buf.cpu()[valid],
                           K.pack_frag_a_ref(o.view(Ssuf, H * D).cpu())[valid])


@pytest.mark.parametrize('splits', [0, 1, 14])
@pytest.mark.parametrize('spike', ['late', 'early'])
def test_attention_decode_score_jump(K, cuda, splits, spike):
    """Scores of one 64-key tile far above the others (~900 in the exp2
    domain).  'late': the jump comes after the rows fixed their exp2
    reference on an earlier tile; with one key range (splits=1, the
    transposed kernel) that sends the workgroup through its second pass
    (exact row maxima), with 14 ranges (the 4-wave kernel) the online
    rescale takes it.  'early': the first tile holds the peak and the later
    keys underflow towards zero."""
    announce(f'attention decode score jump {spike} splits={splits}')
    P, Ssuf, H, D = 816, 51, 8, 256
    T = P + Ssuf
    q = randn((1, Ssuf, H, D), 96)
    cache_k = randn((1, T, D), 97)
    cache_v = randn((1, T, D), 98)
    lo = 320 if spike == 'late' else 0
    # keys lo .. lo + 63 aligned with every query of token 0, head 0
    cache_k[0, lo:lo + 64] = (q[0, 0, 0].float() * 40.0).bfloat16()
    o = torch.empty(1, Ssuf, H, D, dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros(1, D, 872, dtype=torch.bfloat16)  # value cache, 8-aligned rows
    vc[:, :, :T] = cache_v.transpose(1, 2)
    K.mqa_attention(q.to(cuda), cache_k.to(cuda), vc.to(cuda), o,
                    kv_splits=splits, v_transposed=True)
    ref = sdpa_ref(q.double().transpose(1, 2), cache_k.double()[:, None],
                   cache_v.double()[:, None]).transpose(1, 2)
    assert torch.isfinite(o.float()).all()
    assert rel_err(o, ref) <= REL_TOL


def test_attention_siglip_packed(K, cuda):
    announce('attention siglip packed hd=72')
    nv, S, H, D = 3, 256, 16, 72
    qkv = randn((nv * S, 3 * H * D), 95)
    out = torch.empty(nv * S, H * D, dtype=torch.bfloat16, device=cuda)
    K.mha_packed_qkv(qkv.to(cuda), out, nv, S, H, D)
    t = qkv.float().view(nv, S, 3, H, D).permute(2, 0, 3, 1, 4)
    ref = F.scaled_dot_product_attention(t[0], t[1], t[2])
    ref = ref.transpose(1, 2).reshape(nv * S, H * D)
    assert rel_err(out, ref) <= REL_TOL


# ---------------------------------------------------------------------------
# Data movement
# ---------------------------------------------------------------------------
def test_im2col_and_patch_embed(K, cuda):
    announce('im2col + patch embed gemm')
    imgs = torch.rand(3, 3, 224, 224, generator=gen(100)) * 2 - 1
    w = randn((1152, 3, 14, 14), 101, std=0.02)
    b = randn((1152,), 102, std=0.1)
    kpad = 592
    wp = torch.zeros(1152, kpad, dtype=torch.bfloat16)
    wp[:, :588] = w.view(1152, -1)
    patches = K.im2col_patches(imgs.to(cuda), 14, kpad)
    out = K.gemm(patches, wp.to(cuda), bias=b.to(cuda))
    ref = F.conv2d(imgs.bfloat16().float(), w.float(), b.float(), stride=14)
    ref = ref.flatten(2).transpose(1, 2).reshape(768, 1152)
    assert rel_err(out, ref) <= REL_TOL


def test_embed_tokens_and_copy_rows(K, cuda):
    announce('embed tokens / copy rows')
    table = randn((1000, 2048), 110)
    ids = torch.randint(0, 1000, (2, 48), generator=gen(111))
    out = torch.zeros(2, 100, 2048, dtype=torch.bfloat16, device=cuda)
    K.embed_tokens(table.to(cuda), ids.to(cuda), out.view(-1, 2048)[52:],
                   scale=2048 ** 0.5, row_group=48, row_group_stride=100)
    ref = (table[ids].float() * 2048 ** 0.5).bfloat16()
    assert torch.equal(out[:, 52:].cpu(), ref)
    src = randn((2, 64), 112)
    dst = torch.zeros(2, 10, 64, dtype=torch.bfloat16, device=cuda)
    K.copy_rows(src.to(cuda), dst.view(-1, 64), row_group=1,
                dst_group_stride=10)
    assert torch.equal(dst[:, 0].cpu(), src)
    assert dst[:, 1:].abs().max().item() == 0.0


@pytest.mark.parametrize('place', [False, True])
def test_decode_attention_prefetch_changes_nothing(cuda, place):
    """The expert decode attention with prefetch ranges (extra workgroups
    reading the next GEMMs' fragment-major weights): bitwise the output
    without them, the prefetched buffers untouched."""
    from fluxvla_amd import kernels as Kk
    announce(f'decode attention with prefetch place={place}')
    g = torch.Generator().manual_seed(70)
    B, Sq, H, D, S, T = 1, 51, 8, 256, 816, 872
    q = torch.randn(B, Sq, H, D, generator=g).bfloat16().to(cuda)
    k = torch.randn(B, T, D, generator=g).bfloat16().to(cuda)
    vt = torch.randn(B, D, T, generator=g).bfloat16().to(cuda)
    kgrp = torch.zeros(B, S + Sq, dtype=torch.int32, device=cuda)
    kgrp[:, S + 1:] = 1
    qgrp = torch.ones(B, Sq, dtype=torch.int32, device=cuda)
    qgrp[:, 0] = 0
    ws = [Kk.FragB.pack((torch.randn(n, kk, generator=g) * 0.02).bfloat16().to(cuda))
          for n, kk in ((1024, 2048), (4096, 1024), (4096, 1024), (1024, 4096),
                        (2560, 1024))]
    before = [w.buf.clone() for w in ws]
    o1 = torch.empty_like(q)
    o2 = torch.empty_like(q)
    Kk.mqa_attention(q, k[:, :S + Sq], vt, o1, kgrp=kgrp, qgrp=qgrp,
                     v_transposed=True)
    Kk.mqa_attention(q, k[:, :S + Sq], vt, o2, kgrp=kgrp, qgrp=qgrp,
                     v_transposed=True, prefetch=ws, prefetch_place=place)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert all(torch.equal(a, w.buf) for a, w in zip(before, ws))


@pytest.mark.parametrize('m,n,k', [(768, 1152, 4304), (768, 3456, 1152), (816, 2048, 2048),
                                   (130, 200, 72)])
def test_plain_epilogue_build_is_bitwise_generic(K, cuda, m, n, k):
    """The tile kernel's plain-epilogue build (PLAIN with bias, fp32 bias,
    activation, residual) against the generic epilogue on the same call
    (forced by an identity row group: out row m = m), bit for bit, and
    against an fp32 reference."""
    announce(f'plain epilogue build m={m} n={n} k={k}')
    from fluxvla_amd._lib import ACT_GELU_TANH, ACT_NONE
    a = randn((m, k), 80).to(cuda)
    w = randn((n, k), 81, std=0.02).to(cuda)
    b = randn((n,), 82, std=0.5).to(cuda)
    bf = torch.randn(n, generator=gen(83)).to(cuda)
    res = randn((m, n), 84).to(cuda)
    for kw in (dict(bias=b, residual=res), dict(bias_f32=bf, act=ACT_GELU_TANH),
               dict(bias=b, bias_f32=bf, act=ACT_NONE, residual=res)):
        fast = K.gemm(a, w, **kw)
        generic = K.gemm(a, w, row_group=m, row_group_stride=m, **kw)
        assert torch.equal(fast, generic)
        ref = a.float() @ w.float().t()
        if 'bias' in kw:
            ref = ref + b.float()
        if 'bias_f32' in kw:
            ref = ref + bf
        if kw.get('act') == ACT_GELU_TANH:
            ref = F.gelu(ref, approximate='tanh')
        if 'residual' in kw:
            ref = ref + res.float()
        assert rel_err(fast, ref) <= REL_TOL


@pytest.mark.parametrize('m,n,k,split_k', [(816, 2048, 16384, 0), (200, 256, 4096, 2)])
def test_plain_reduce_build_is_bitwise_generic(K, cuda, m, n, k, split_k):
    """The split-K reduce's plain-epilogue build (behind the wide kernel over
    8 K ranges: the prefix down projection; behind split tiles) against the
    generic epilogue (forced by an identity row group), bit for bit, with
    the row sums of squares handed over; and against an fp32 reference."""
    announce(f'plain reduce build m={m} n={n} k={k} split_k={split_k}')
    a = randn((m, k), 90).to(cuda)
    w = randn((n, k), 91, std=0.01).to(cuda)
    b = randn((n,), 92, std=0.5).to(cuda)
    res = randn((m, n), 93).to(cuda)
    outs = []
    for kw in ({}, dict(row_group=m, row_group_stride=m)):
        x = res.clone()
        ss = torch.zeros(K.ss_parts(n), m, device=cuda)
        K.gemm(a, w, out=x, bias=b, residual=x, ss_out=ss if split_k == 0 else None,
               split_k=split_k, **kw)
        outs.append((x, ss))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    ref = a.float() @ w.float().t() + b.float() + res.float()
    assert rel_err(outs[0][0], ref) <= REL_TOL


@pytest.mark.parametrize('m,n,k', [(51, 1024, 2048), (51, 1024, 4096), (17, 1000, 1000)])
def test_plain_epilogue_build_skinny_gate_frag(K, cuda, m, n, k):
    """The skinny kernel's plain-epilogue build (the bs=1 expert's O and
    down projections: residual, per-row gate, fragment-major copy, bias)
    against the generic epilogue on the same call (forced by an identity
    row group), bit for bit in both outputs, and against fp32."""
    announce(f'plain epilogue build skinny m={m} n={n} k={k}')
    a = randn((m, k), 94).to(cuda)
    w = randn((n, k), 95, std=0.02).to(cuda)
    b = randn((n,), 96, std=0.5).to(cuda)
    res = randn((m, n), 97).to(cuda)
    gate = randn((m, n), 98, std=0.5).to(cuda)
    outs = []
    for kw in ({}, dict(row_group=m, row_group_stride=m)):
        x = res.clone()
        cf = K.FragA.empty(n, cuda).rows(m) if n % 32 == 0 else None
        K.gemm(a, w, out=x, bias=b, residual=x, gate=gate, c_frag=cf, **kw)
        outs.append((x, cf))
    assert torch.equal(outs[0][0], outs[1][0])
    if outs[0][1] is not None:
        assert torch.equal(outs[0][1].buf, outs[1][1].buf)
    ref = (a.float() @ w.float().t() + b.float()) * gate.float() + res.float()
    assert rel_err(outs[0][0], ref) <= REL_TOL
