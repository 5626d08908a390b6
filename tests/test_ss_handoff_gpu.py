"""Row sums of squares handed from one GEMM to the next (ss_out / ss_in).

A PLAIN GEMM with ``ss_out`` also writes, per row and 64-column block, the
sum of squares of its outputs as stored (bf16-rounded); a rownorm GEMM with
``ss_in`` takes the sum of squares of its A rows from those parts instead of
summing them in its K loop.  Pinned against float64 sums of the stored
outputs (producer), against the float64 reference of the fused op
(consumer, the bf16 op bar), and against the same GEMM summing A itself
(they differ only in fp32 summation order).
"""
import pytest
import torch
import torch.nn.functional as F

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


def block_sumsq(x, parts):
    """float64 [parts, M]: sums of squares of x's 64-column blocks."""
    xd = x.double().cpu()
    m, n = xd.shape
    out = torch.zeros(parts, m, dtype=torch.float64)
    for p in range(parts):
        out[p] = xd[:, 64 * p:64 * (p + 1)].pow(2).sum(1)
    return out


def produce(K, cuda, m, k, n, seed):
    """x = res + a @ w^T through a PLAIN GEMM that also writes ss_out."""
    a = randn((m, k), seed, std=1.0)
    w = randn((n, k), seed + 1, std=0.03)
    res = randn((m, n), seed + 2)
    x = res.to(cuda)
    parts = K.ss_parts(n)
    ss = torch.full((parts, m + 3), float('nan'), device=cuda)
    K.gemm(a.to(cuda), w.to(cuda), out=x, residual=x, ss_out=ss)
    return x, ss, parts


@pytest.mark.parametrize('m,k,n', [(816, 2048, 2048), (300, 512, 1000),
                                   (65, 256, 72)])
def test_ss_out_block_sums(K, cuda, m, k, n):
    announce(f'ss_out m={m} k={k} n={n}')
    x, ss, parts = produce(K, cuda, m, k, n, 10)
    ref = block_sumsq(x, parts)
    got = ss[:, :m].double().cpu()
    assert torch.isfinite(got).all()
    assert ((got - ref).abs() <= 1e-5 * ref.abs() + 1e-6).all()
    # columns past m are not written
    assert torch.isnan(ss[:, m:].cpu()).all()


def within_ulp(got, own):
    """Equal up to one bf16 rounding step per element: the two GEMMs differ
    only in the fp32 summation order of the RMS factor, which can flip the
    final bf16 rounding."""
    g, o = got.double().cpu(), own.double().cpu()
    return ((g - o).abs() <= 2.0**-7 * o.abs() + 1e-6 * o.abs().max()).all()


def rms(x, eps=1e-6):
    xd = x.double().cpu()
    return torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps)


@pytest.mark.parametrize('m,n', [(816, 16384), (816, 512), (300, 384)])
def test_ss_in_geglu(K, cuda, m, n):
    """Consumer: the wide 256 x 256 GeGLU kernel (m=816, n=16384) and the
    tiled one, against float64 and against the in-kernel sums."""
    announce(f'ss_in geglu m={m} n={n}')
    hid = 2048 if m == 816 else 512
    x, ss, _ = produce(K, cuda, m, 256, hid, 20)
    wg = randn((n, hid), 23, std=0.02).to(cuda)
    wu = randn((n, hid), 24, std=0.02).to(cuda)
    got = K.gemm_geglu(x, wg, wu, rownorm_eps=1e-6, ss_in=ss[:, :m])
    own = K.gemm_geglu(x, wg, wu, rownorm_eps=1e-6)
    xn = x.double().cpu() * rms(x)
    ref = (F.gelu(xn @ wg.double().cpu().t(), approximate='tanh') *
           (xn @ wu.double().cpu().t()))
    assert rel_err(got, ref) <= REL_TOL
    assert within_ulp(got, own)


@pytest.mark.parametrize('split', [0, 2])
def test_ss_in_plain_and_split(K, cuda, split):
    """Consumer on the tiled PLAIN path, one pass and split-K (the handed
    sums ride with split 0 only)."""
    announce(f'ss_in plain split_k={split}')
    m, hid, n = 400, 4096, 384
    x, ss, _ = produce(K, cuda, m, 128, hid, 30)
    w = randn((n, hid), 33, std=0.02).to(cuda)
    got = K.gemm(x, w, rownorm_eps=1e-6, ss_in=ss[:, :m], split_k=split)
    own = K.gemm(x, w, rownorm_eps=1e-6, split_k=split)
    ref = (x.double().cpu() * rms(x)) @ w.double().cpu().t()
    assert rel_err(got, ref) <= REL_TOL
    assert within_ulp(got, own)


def test_ss_in_qkv_rope(K, cuda):
    """Consumer on the QKV + RoPE epilogue (the next layer's projection)."""
    announce('ss_in qkv_rope')
    m, hid, nq, hd = 816, 2048, 8, 256
    x, ss, _ = produce(K, cuda, m, 256, hid, 40)
    w = randn(((nq + 2) * hd, hid), 43, std=0.02).to(cuda)
    pos = torch.arange(m, dtype=torch.int32, device=cuda)
    rope = K.rope_table(m + 8, hd, device=cuda)
    outs = []
    for s_in in (ss[:, :m], None):
        q = torch.empty(m, nq * hd, dtype=torch.bfloat16, device=cuda)
        kk = torch.empty(m, hd, dtype=torch.bfloat16, device=cuda)
        vv = torch.empty(m, hd, dtype=torch.bfloat16, device=cuda)
        K.gemm_qkv_rope(x, w, rope, pos, q, kk, vv, nq, hd, rownorm_eps=1e-6,
                        ss_in=s_in)
        outs.append((q, kk, vv))
    for got, own in zip(outs[0], outs[1]):
        assert within_ulp(got, own)


def test_ss_args_rejected(K, cuda):
    """ss_in without rownorm and ss_out on a skinny (M <= 64) or non-PLAIN
    GEMM are argument errors, not silent fallbacks."""
    a = randn((32, 64), 50).to(cuda)
    w = randn((64, 64), 51).to(cuda)
    ss = torch.zeros(1, 128, device=cuda)
    with pytest.raises(ValueError):
        K.gemm(a, w, ss_in=ss)
    with pytest.raises(Exception):
        K.gemm(a, w, ss_out=ss)


@pytest.mark.parametrize('n', [1024, 2048])
def test_ss_in_and_ss_out_in_one_gemm(K, cuda, n):
    """A rownorm PLAIN GEMM that reads handed-over sums (ss_in) and hands its
    own output's sums on (ss_out, with a residual): the tile build with both
    row-sum paths.  Against the same call summing A's squares itself, and
    the handed-on sums against the stored rows."""
    announce(f'ss_in + ss_out plain n={n}')
    m, hid = 816, 2048
    x, ss, _ = produce(K, cuda, m, 256, hid, 50)
    w = randn((n, hid), 53, std=0.02).to(cuda)
    res = randn((m, n), 54).to(cuda)
    outs = []
    for s_in in (ss[:, :m], None):
        y = res.clone()
        # one row stride for both (ss_ld)
        so = torch.full((K.ss_parts(n), m + 3), float('nan'), device=cuda)
        K.gemm(x, w, out=y, residual=y, rownorm_eps=1e-6, ss_in=s_in, ss_out=so)
        outs.append((y, so))
    (y, so), (y_own, _) = outs
    ref = (x.double().cpu() * rms(x)) @ w.double().cpu().t() + res.double().cpu()
    assert rel_err(y, ref) <= REL_TOL
    assert within_ulp(y, y_own)
    want = block_sumsq(y, K.ss_parts(n))
    got = so[:, :m].double().cpu()
    assert ((got - want).abs() <= 1e-5 * want.abs() + 1e-6).all()
