"""The 256 x 256 wide GEMM kernel on PLAIN and QKV + RoPE epilogues.

The planner only picks it for large problems (>= 192 of its tiles and
K >= 2048: batched prefixes), so these tests run at such sizes and check a
sample of rows -- the first and last rows of the tiles and of the problem --
against CPU references (fp32 GEMMs; RoPE in float64).  Bar: the bf16 op bar,
max relative error <= 1e-2.
"""
import pytest
import torch

from tests.conftest import announce

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2


def rel_err(out, ref):
    out = out.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return ((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def randn(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)


@pytest.fixture(scope='module')
def K():
    from fluxvla_amd import kernels
    kernels._lib.load()
    return kernels


def sample_rows(m):
    rows = {0, 1, 127, 128, 255, 256, 511, m // 2, m - 257, m - 256, m - 2, m - 1}
    return torch.tensor(sorted(r for r in rows if 0 <= r < m))


@pytest.mark.parametrize('rownorm', [False, True])
def test_wide_plain_bias_residual(K, cuda, rownorm):
    """M=6528 (8 prefixes), N=2048, K=2048: 26 x 8 = 208 wide tiles."""
    announce(f'wide plain m=6528 rownorm={rownorm}')
    m, n, k = 6528, 2048, 2048
    a = randn((m, k), 1)
    w = randn((n, k), 2, std=0.02)
    b = randn((n,), 3, std=0.5)
    res = randn((m, n), 4)
    x = res.to(cuda)
    parts = K.ss_parts(n)
    ss = torch.zeros(parts, m, device=cuda)
    K.gemm(a.to(cuda), w.to(cuda), out=x, bias=b.to(cuda), residual=x,
           rownorm_eps=1e-6 if rownorm else None, ss_out=ss)
    rows = sample_rows(m)
    af = a[rows].float()
    if rownorm:
        af = af * torch.rsqrt(af.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = af @ w.float().t() + b.float() + res[rows].float()
    got = x.cpu()[rows]
    assert rel_err(got, ref) <= REL_TOL
    # row sums of squares of the stored bf16 rows, per 64-column block
    gd = got.double()
    for p in range(parts):
        want = gd[:, 64 * p:64 * (p + 1)].pow(2).sum(1)
        have = ss.cpu()[p, rows].double()
        assert ((have - want).abs() <= 1e-5 * want + 1e-6).all()


def test_wide_plain_full_output(K, cuda):
    """Every row of a wide-kernel GEMM (M=6528, N=2048, K=4096) against an
    fp32 GEMM of the same bf16 operands on the GPU."""
    announce('wide plain full output m=6528 k=4096')
    m, n, k = 6528, 2048, 4096
    a = randn((m, k), 11).to(cuda)
    w = randn((n, k), 12, std=0.02).to(cuda)
    got = K.gemm(a, w)
    ref = a.float() @ w.float().t()
    assert rel_err(got, ref) <= REL_TOL


def test_wide_qkv_rope(K, cuda):
    """QKV + RoPE at M=6144, N=2560 (24 x 10 = 240 wide tiles), rownorm."""
    announce('wide qkv_rope m=6144')
    from tests.test_kernels_gpu import interleave_perm, rope_ref
    m, k, nq, hd = 6144, 2048, 8, 256
    x = randn((m, k), 21, std=1.5)
    wq = randn((nq * hd, k), 22, std=0.02)
    wk = randn((hd, k), 23, std=0.02)
    wv = randn((hd, k), 24, std=0.02)
    perm = interleave_perm(hd)
    w = torch.cat([wq.view(nq, hd, k)[:, perm].reshape(nq * hd, k), wk[perm], wv], 0)
    pos = torch.arange(m, dtype=torch.int32) % 900
    rope = K.rope_table(1000, hd, device=cuda)
    q = torch.empty(m, nq * hd, dtype=torch.bfloat16, device=cuda)
    kk = torch.empty(m, hd, dtype=torch.bfloat16, device=cuda)
    vv = torch.empty(m, hd, dtype=torch.bfloat16, device=cuda)
    K.gemm_qkv_rope(x.to(cuda), w.contiguous().to(cuda), rope, pos.to(cuda), q, kk, vv,
                    nq, hd, rownorm_eps=1e-6)
    rows = sample_rows(m)
    xf = x[rows].double()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    p = pos[rows]
    rq = rope_ref((xn @ wq.double().t()).view(-1, nq, hd), p, hd)
    rk = rope_ref((xn @ wk.double().t()).view(-1, 1, hd), p, hd)
    rv = xn @ wv.double().t()
    inv = torch.argsort(perm)
    assert rel_err(q.cpu()[rows].view(-1, nq, hd)[:, :, inv], rq) <= REL_TOL
    assert rel_err(kk.cpu()[rows][:, inv], rk.view(-1, hd)) <= REL_TOL
    assert rel_err(vv.cpu()[rows], rv) <= REL_TOL


def test_wide_split_k_down(K, cuda):
    """The prefix down projection at bs=1 (M=816, N=2048, K=16384: 32 wide
    tiles) runs the wide kernel over 8 K ranges, then the split-K reduce
    runs the epilogue (residual in place) and the hand-overs: row sums of
    squares of the stored output and its e4m3 copy.  Checked against an
    fp32 GEMM (bf16 op bar), float64 sums and the quantization
    restatement of the stored output, and against the one-pass 64 x 128
    kernel (split_k=1) within one bf16 rounding step."""
    announce('wide split-K down m=816 k=16384')
    from tests.test_fp8_gpu import quant_blocks_ref
    m, n, k = 816, 2048, 16384
    a = randn((m, k), 31)
    w = randn((n, k), 32, std=0.01)
    res = randn((m, n), 33)
    parts = K.ss_parts(n)
    outs = []
    for sk in (0, 1):
        x = res.to(cuda)
        ss = torch.zeros(parts, m, device=cuda)
        a8 = K.Fp8Act.empty(m, n, cuda)
        K.gemm(a.to(cuda), w.to(cuda), out=x, residual=x, ss_out=ss, a8_out=a8,
               split_k=sk)
        outs.append((x.cpu(), ss.cpu(), a8))
    x, ss, a8 = outs[0]
    ref = a.float() @ w.float().t() + res.float()
    assert rel_err(x, ref) <= REL_TOL
    want = x.double().view(m, parts, 64).pow(2).sum(-1).t()
    assert ((ss.double() - want).abs() <= 1e-5 * want + 1e-6).all()
    q, e = quant_blocks_ref(x)
    assert torch.equal(a8.data.cpu(), q)
    assert torch.equal(a8.scale.cpu()[:, :m].t(), e)
    x1 = outs[1][0]
    assert ((x.double() - x1.double()).abs() <= 2.0**-7 * x1.double().abs() + 1e-3).all()
