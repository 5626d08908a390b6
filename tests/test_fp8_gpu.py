"""fp8 (e4m3) weight GEMMs: the PI0.5 quantized-weight variant, in its two
arithmetics: W8A16 (the default: bf16 activations, the e4m3 weights
converted to bf16 in registers, bf16 MFMA, fp32 accumulation) and W8A8
(opt-in: activations quantized to e4m3 per row and k step).

W8A16 is pinned against float64 a @ dequant(W)^T (exact up to fp32
summation order), and the conversion itself bit for bit: a one-hot A
times weights holding every finite e4m3 byte returns each byte's value.

The reference has no fp8 path, so the W8A8 kernels are pinned two ways:

* exactly, against a float64 restatement of what they compute: the weight
  dequantized from its e4m3 bytes and per-channel scale, and the A values of
  each row and MFMA k step (64 values in the tiled kernel, 128 in the skinny
  one) quantized to e4m3 under one power-of-two scale 2^(e - 127),
  e = E - 8 + (mantissa > 96) from the block maximum's bf16 exponent E and
  7-bit mantissa (the smallest power of two that keeps the block within
  448).  The bar is the bf16 op bar, max relative error <= 1e-2 (what
  remains is fp32 accumulation and the bf16 output rounding);
* by the rounding bound of e4m3 against the unquantized bf16 activations:
  |out - a @ Wq^T| <= 2^-4 (|a| @ |Wq|^T) elementwise (3 mantissa bits give a
  relative rounding error of at most 2^-4 for every quantized value), which
  a wrong block layout or scale convention would violate by orders of
  magnitude.

One scale per (row, step) rather than per 32 values: the block-scaled MFMAs
apply a lane's scale to 16-byte halves held by other lanes of the same row
(measured on gfx950), so a scale shared by the row's lanes is the choice that
makes the product exact without depending on that assignment.
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


def block_ids(k, skinny):
    kk = torch.arange(k)
    return kk // 128 if skinny else kk // 64


def quant_a_ref(a, skinny):
    """float64 values the kernel multiplies: a (bf16 [m, k]) with every
    block (row, k step) quantized to e4m3 under its power-of-two scale."""
    m, k = a.shape
    bid = block_ids(k, skinny)
    nb = int(bid.max()) + 1
    bits = a.view(torch.int16).int() & 0x7FFF           # |a| bf16 bits
    amax = torch.zeros(m, nb, dtype=torch.int32)
    amax.scatter_reduce_(1, bid.expand(m, k), bits, 'amax')
    E, mant = (amax >> 7) & 0xFF, amax & 0x7F
    e = (E - 8 + (mant > 96).int()).clamp(1, 254)
    scale = torch.pow(2.0, (e - 127).double())          # [m, nb]
    sc = scale.gather(1, bid.expand(m, k))
    q = (a.double() / sc).float().to(torch.float8_e4m3fn).double()
    return q * sc


def fp8_weight(K, w, cuda, frag=False, act='e4m3'):
    fw = K.Fp8Weight.quantize(w.to(cuda), act=act)
    wq = fw.dequantize().double().cpu()
    return (fw.pack_frag() if frag else fw), wq


def check_bound(out, a, wq, ref_extra=None):
    """e4m3 rounding bound against the unquantized activations."""
    exact = a.double() @ wq.t()
    bound = (a.double().abs() @ wq.abs().t()) * 2.0**-4
    out = out.detach().double().cpu()
    if ref_extra is not None:
        out = out - ref_extra
    # 1e-2 of the output scale covers the bf16 rounding of the stored result
    slack = 1e-2 * exact.abs().max()
    assert ((out - exact).abs() <= bound + slack).all()


@pytest.mark.parametrize('m,n,k', [(300, 384, 512), (816, 640, 2048),
                                   (129, 256, 128)])
def test_fp8_gemm_tile(K, cuda, m, n, k):
    announce(f'fp8 gemm tile m={m} n={n} k={k}')
    a = randn((m, k), 100, std=1.5)
    fw, wq = fp8_weight(K, randn((n, k), 101, std=0.02), cuda)
    bias = randn((n,), 102, std=0.5)
    res = randn((m, n), 103)
    out = K.gemm(a.to(cuda), fw, bias=bias.to(cuda), residual=res.to(cuda))
    extra = bias.double() + res.double()
    ref = quant_a_ref(a, skinny=False) @ wq.t() + extra
    assert rel_err(out, ref) <= REL_TOL
    check_bound(out, a, wq, ref_extra=extra)


@pytest.mark.parametrize('m,n,k', [(51, 2560, 1024), (50, 1024, 2048),
                                   (51, 1024, 4096), (1, 256, 128)])
def test_fp8_gemm_skinny_frag(K, cuda, m, n, k):
    announce(f'fp8 gemm skinny m={m} n={n} k={k}')
    a = randn((m, k), 110, std=1.5)
    fw, wq = fp8_weight(K, randn((n, k), 111, std=0.02), cuda, frag=True)
    af = K.pack_frag(a.to(cuda), K.FragA.empty(k, cuda).rows(m))
    res = randn((m, n), 112)
    out = K.gemm(af, fw, residual=res.to(cuda))
    ref = quant_a_ref(a, skinny=True) @ wq.t() + res.double()
    assert rel_err(out, ref) <= REL_TOL
    check_bound(out, a, wq, ref_extra=res.double())


@pytest.mark.parametrize('m,skinny', [(51, True), (200, False)])
def test_fp8_gemm_geglu_rownorm(K, cuda, m, skinny):
    announce(f'fp8 gemm geglu rownorm m={m} skinny={skinny}')
    n, k = 512, 1024
    a = randn((m, k), 120, std=2.0)
    gw, gq = fp8_weight(K, randn((n, k), 121, std=0.02), cuda, frag=skinny)
    uw, uq = fp8_weight(K, randn((n, k), 122, std=0.02), cuda, frag=skinny)
    ad = a.to(cuda)
    if skinny:
        ad = K.pack_frag(ad, K.FragA.empty(k, cuda).rows(m))
    out = K.gemm_geglu(ad, gw, uw, rownorm_eps=1e-6)
    aq = quant_a_ref(a, skinny=skinny)
    r = torch.rsqrt(a.double().pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = F.gelu((aq @ gq.t()) * r, approximate='tanh') * ((aq @ uq.t()) * r)
    assert rel_err(out, ref) <= REL_TOL


def test_fp8_quantization_edge_blocks(K, cuda):
    """Blocks at the scale boundaries: a block maximum with mantissa 96 and
    97 (exactly 448 2^s and just above), all-zero rows, tiny and huge
    magnitudes; the restatement must agree to fp32 accumulation."""
    announce('fp8 gemm edge blocks')
    m, n, k = 96, 128, 256
    a = randn((m, k), 130)
    a[0] = 0.0
    a[1, :32] = 1.75                    # 1.75 = 1 + 96/128: e = E - 8
    a[2, :32] = 1.7578125               # 1 + 97/128: e = E - 7
    a[3] = randn((k,), 131) * 1e-30
    a[4] = randn((k,), 132) * 1e30
    a[5, 5] = 448.0
    fw, wq = fp8_weight(K, randn((n, k), 133, std=0.05), cuda)
    out = K.gemm(a.to(cuda), fw, out_f32=True)
    aq = quant_a_ref(a, skinny=False)
    ref = aq @ wq.t()
    mass = aq.abs() @ wq.abs().t()      # sum of |products| per output
    got = out.double().cpu()
    # fp32 output, each row against its own scale.  The fp8 MFMA adds a
    # step's products at a precision set by the largest of them: next to the
    # 448 of row 5 the others lose low-order bits (measured ~1e-4 of the
    # row's mass), far below any layout or scale mistake (a factor of 2).
    for row in range(m):
        scale = mass[row].max().item()
        if scale == 0.0:
            assert got[row].abs().max().item() == 0.0
        else:
            assert (got[row] - ref[row]).abs().max().item() <= 1e-3 * scale


def test_fp8_weight_quantization_and_layout(K, cuda):
    """Fp8Weight: per-channel scale = max|row| / 448 (the largest entry of
    every row maps to 448 exactly), dequantization error within e4m3's
    half-ulp, and the fragment-major packing is a permutation of the bytes
    placing (n, k) where fvx_gemm_desc documents it."""
    announce('fp8 weight quantization and packing')
    w = randn((64, 256), 140, std=0.03)
    fw = K.Fp8Weight.quantize(w.to(cuda), act='e4m3')
    assert torch.allclose(fw.scale.cpu(), w.float().abs().amax(1) / 448.0)
    wd = fw.dequantize().cpu()
    assert ((wd - w.float()).abs() <= 2.0**-4 * w.float().abs() +
            fw.scale.cpu()[:, None] * 2.0**-10).all()
    q = fw.data.cpu()
    assert (q.view(torch.float8_e4m3fn).float().abs().amax(1) == 448.0).all()
    fb = fw.pack_frag().data.cpu()
    n, kk = torch.meshgrid(torch.arange(64), torch.arange(256), indexing='ij')
    r = kk % 128
    pos = (((n // 16) * 2 + kk // 128) * 2048 + ((r // 8) % 4 * 16 + n % 16) * 32
           + (r // 32) * 8 + kk % 8)
    assert torch.equal(fb[pos.reshape(-1)].view(64, 256), q)


def sample_rows(m):
    rows = {0, 1, 127, 128, 255, 256, m // 2, m - 257, m - 256, m - 2, m - 1}
    return torch.tensor(sorted(r for r in rows if 0 <= r < m))


def test_fp8_wide_geglu(K, cuda):
    """The wide fp8 kernel (256 x 2 x 128 tiles; the prefix gate/up shape,
    512 tiles) on sampled rows, against the restatement with per-(row,
    64-k) activation scales and against the e4m3 rounding bound."""
    announce('fp8 wide geglu m=816 n=16384 k=2048')
    m, n, k = 816, 16384, 2048
    a = randn((m, k), 150, std=1.5)
    gw, gq = fp8_weight(K, randn((n, k), 151, std=0.02), cuda)
    uw, uq = fp8_weight(K, randn((n, k), 152, std=0.02), cuda)
    out = K.gemm_geglu(a.to(cuda), gw, uw, rownorm_eps=1e-6)
    rows = sample_rows(m)
    aq = quant_a_ref(a[rows], skinny=False)
    r = torch.rsqrt(a[rows].double().pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = F.gelu((aq @ gq.t()) * r, approximate='tanh') * ((aq @ uq.t()) * r)
    assert rel_err(out.cpu()[rows], ref) <= REL_TOL


def test_fp8_wide_plain(K, cuda):
    """The wide fp8 kernel on a PLAIN GEMM with bias and residual (M=6528,
    N=2048, K=2048: 208 tiles), sampled rows."""
    announce('fp8 wide plain m=6528 n=2048 k=2048')
    m, n, k = 6528, 2048, 2048
    a = randn((m, k), 160, std=1.5)
    fw, wq = fp8_weight(K, randn((n, k), 161, std=0.02), cuda)
    bias = randn((n,), 162, std=0.5)
    res = randn((m, n), 163)
    out = K.gemm(a.to(cuda), fw, bias=bias.to(cuda), residual=res.to(cuda))
    rows = sample_rows(m)
    extra = bias.double() + res[rows].double()
    ref = quant_a_ref(a[rows], skinny=False) @ wq.t() + extra
    got = out.cpu()[rows]
    assert rel_err(got, ref) <= REL_TOL
    check_bound(got, a[rows], wq, ref_extra=extra)


def quant_blocks_ref(x):
    """CPU restatement of the e4m3 hand-over copy of a bf16 matrix [m, n]:
    per row and 64-column block, e = E - 8 + (mantissa > 96) of the block's
    largest |value| (clamped to [1, 254]), q = e4m3(x / 2^(e - 127))."""
    m, n = x.shape
    bits = (x.view(torch.int16).int() & 0x7FFF).view(m, n // 64, 64)
    amax = bits.amax(-1)
    E, mant = (amax >> 7) & 0xFF, amax & 0x7F
    e = (E - 8 + (mant > 96).int()).clamp(1, 254)
    sc = torch.pow(2.0, (e - 127).double()).repeat_interleave(64, 1)
    q = (x.double() / sc).float().to(torch.float8_e4m3fn)
    return q.view(torch.uint8), e.to(torch.uint8)


@pytest.mark.parametrize('m,n,k,geglu', [(300, 1024, 512, False), (816, 16384, 2048, True)])
def test_fp8_handover_copy_exact(K, cuda, m, n, k, geglu):
    """The e4m3 copy a GEMM epilogue writes (a8_out) is byte for byte the
    quantization of its stored bf16 output, exponents included."""
    announce(f'fp8 hand-over copy m={m} n={n} geglu={geglu}')
    a = randn((m, k), 170).to(cuda)
    w = randn((n, k), 171, std=0.03).to(cuda)
    a8 = K.Fp8Act.empty(m, n, cuda)
    if geglu:
        w2 = randn((n, k), 172, std=0.03).to(cuda)
        out = K.gemm_geglu(a, w, w2, rownorm_eps=1e-6, a8_out=a8)
    else:
        out = K.gemm(a, w, a8_out=a8)
    rows = sample_rows(m)
    q, e = quant_blocks_ref(out.cpu()[rows])
    assert torch.equal(a8.data.cpu()[rows], q)
    assert torch.equal(a8.scale.cpu()[:, rows].t(), e)


def test_fp8_handover_consumer_identical(K, cuda):
    """The fp8 wide GEMM reading the e4m3 copy of A (a8) gives bitwise the
    result of the same GEMM quantizing the bf16 A itself: the same values
    and exponents feed the same MFMAs.  Gate/up shape with handed-over row
    sums, and a PLAIN shape (M=6528)."""
    announce('fp8 hand-over consumer == self-quantizing')
    for m, k, n, geglu in ((816, 2048, 16384, True), (6528, 2048, 2048, False)):
        a0 = randn((m, 256), 180).to(cuda)
        w0 = randn((k, 256), 181, std=0.05).to(cuda)
        x = torch.empty(m, k, dtype=torch.bfloat16, device=cuda)
        ss = torch.zeros(K.ss_parts(k), m, device=cuda)
        a8 = K.Fp8Act.empty(m, k, cuda)
        K.gemm(a0, w0, out=x, ss_out=ss, a8_out=a8)      # producer
        fw = K.Fp8Weight.quantize(randn((n, k), 182, std=0.02).to(cuda), act='e4m3')
        if geglu:
            fu = K.Fp8Weight.quantize(randn((n, k), 183, std=0.02).to(cuda),
                                      act='e4m3')
            got = K.gemm_geglu(x, fw, fu, rownorm_eps=1e-6, ss_in=ss, a8=a8)
            own = K.gemm_geglu(x, fw, fu, rownorm_eps=1e-6, ss_in=ss)
        else:
            res = randn((m, n), 184).to(cuda)
            got = K.gemm(x, fw, residual=res, a8=a8)
            own = K.gemm(x, fw, residual=res)
        assert torch.equal(got, own)


def test_fp8_wide_split_k_down(K, cuda):
    """The fp8 prefix down projection at bs=1 (M=816, N=2048, K=16384, fp8
    weights): the fp8 wide kernel over 8 K ranges, partials scaled by the
    weight scales, then the split-K reduce (residual in place, row sums and
    e4m3 copy of the output).  A both ways: the e4m3 copy handed over by a
    producer (a8) and bf16 quantized in the kernel.  Against the float64
    quantization restatement (bf16 op bar), and the hand-overs against the
    stored output."""
    announce('fp8 wide split-K down m=816 k=16384')
    m, n, k = 816, 2048, 16384
    a0 = randn((m, 512), 190)
    w0 = randn((k, 512), 191, std=0.05).to(cuda)
    fw, wq = fp8_weight(K, randn((n, k), 192, std=0.01), cuda)
    res = randn((m, n), 193)
    # producer: A (bf16) and its e4m3 copy
    a = torch.empty(m, k, dtype=torch.bfloat16, device=cuda)
    a8 = K.Fp8Act.empty(m, k, cuda)
    K.gemm(a0.to(cuda), w0, out=a, a8_out=a8)
    rows = sample_rows(m)
    ac = a.cpu()
    ref = quant_a_ref(ac[rows], skinny=False) @ wq.t() + res[rows].double()
    parts = K.ss_parts(n)
    for use_a8 in (True, False):
        x = res.to(cuda)
        ss = torch.zeros(parts, m, device=cuda)
        o8 = K.Fp8Act.empty(m, n, cuda)
        K.gemm(a, fw, out=x, residual=x, ss_out=ss, a8_out=o8,
               a8=a8 if use_a8 else None)
        got = x.cpu()
        assert rel_err(got[rows], ref) <= REL_TOL
        want = got.double().view(m, parts, 64).pow(2).sum(-1).t()
        assert ((ss.cpu().double() - want).abs() <= 1e-5 * want + 1e-6).all()
        q, e = quant_blocks_ref(got)
        assert torch.equal(o8.data.cpu(), q)
        assert torch.equal(o8.scale.cpu()[:, :m].t(), e)


# ---------------------------------------------------------------------------
# W8A16 (the default fp8 arithmetic)
# ---------------------------------------------------------------------------
# fp32 accumulation + the bf16 output rounding (half an ulp of an element
# up to twice the largest |ref| binade: ~2^-8 of max |ref|); an e4m3 rounding
# of the activations (2^-4 relative) would exceed it by an order of magnitude
W16_TOL = 5e-3


def test_w8a16_conversion_exact(K, cuda):
    """Weights holding every finite e4m3 byte (scale 1) times a one-hot A
    (fp32 output): out[m, n] is exactly the e4m3 value of W[n, m], subnormals
    and signed zeros included -- through the tiled (M = 128) and the skinny
    fragment-major (M = 64) kernels."""
    announce('w8a16 e4m3 -> bf16 conversion exact')
    codes = torch.tensor([c for c in range(256) if c & 0x7F != 0x7F],
                         dtype=torch.uint8)                       # 254 finite
    n, k = 256, 128
    data = torch.zeros(n, k, dtype=torch.uint8)
    for r in range(n):
        data[r] = codes[(torch.arange(k) + 7 * r) % len(codes)]
    fw = K.Fp8Weight(data.to(cuda), torch.ones(n, device=cuda), n, k)
    want = data.view(torch.float8_e4m3fn).float().t()              # [k, n]
    a = torch.eye(k, dtype=torch.bfloat16, device=cuda)
    out = K.gemm(a, fw, out_f32=True)
    assert torch.equal(out.cpu(), want)
    for r0 in (0, 64):
        af = K.pack_frag(a[r0:r0 + 64], K.FragA.empty(k, cuda).rows(64))
        o = K.gemm(af, fw.pack_frag(), out_f32=True)
        assert torch.equal(o.cpu(), want[r0:r0 + 64])


@pytest.mark.parametrize('m,n,k', [(300, 384, 512), (816, 2560, 2048),
                                   (129, 256, 128), (408, 1024, 4096)])
def test_w8a16_gemm_tile(K, cuda, m, n, k):
    announce(f'w8a16 gemm tile m={m} n={n} k={k}')
    a = randn((m, k), 200, std=1.5)
    fw, wq = fp8_weight(K, randn((n, k), 201, std=0.02), cuda, act='bf16')
    bias = randn((n,), 202, std=0.5)
    res = randn((m, n), 203)
    out = K.gemm(a.to(cuda), fw, bias=bias.to(cuda), residual=res.to(cuda))
    ref = a.double() @ wq.t() + bias.double() + res.double()
    assert rel_err(out, ref) <= W16_TOL


@pytest.mark.parametrize('m,n,k', [(51, 2560, 1024), (50, 1024, 2048),
                                   (51, 1024, 4096), (1, 256, 128),
                                   (33, 4096, 1024)])
def test_w8a16_gemm_skinny_frag(K, cuda, m, n, k):
    announce(f'w8a16 gemm skinny m={m} n={n} k={k}')
    a = randn((m, k), 210, std=1.5)
    fw, wq = fp8_weight(K, randn((n, k), 211, std=0.02), cuda, frag=True,
                        act='bf16')
    af = K.pack_frag(a.to(cuda), K.FragA.empty(k, cuda).rows(m))
    res = randn((m, n), 212)
    out = K.gemm(af, fw, residual=res.to(cuda))
    ref = a.double() @ wq.t() + res.double()
    assert rel_err(out, ref) <= W16_TOL


@pytest.mark.parametrize('m,skinny', [(51, True), (200, False), (816, False)])
def test_w8a16_gemm_geglu_rownorm(K, cuda, m, skinny):
    """GeGLU with the fused RMSNorm: skinny, tiled and (M = 816, N = 16384:
    512 tiles) the wide kernel."""
    announce(f'w8a16 gemm geglu rownorm m={m} skinny={skinny}')
    n, k = (16384, 2048) if m == 816 else (512, 1024)
    a = randn((m, k), 220, std=2.0)
    gw, gq = fp8_weight(K, randn((n, k), 221, std=0.02), cuda, frag=skinny,
                        act='bf16')
    uw, uq = fp8_weight(K, randn((n, k), 222, std=0.02), cuda, frag=skinny,
                        act='bf16')
    ad = a.to(cuda)
    if skinny:
        ad = K.pack_frag(ad, K.FragA.empty(k, cuda).rows(m))
    out = K.gemm_geglu(ad, gw, uw, rownorm_eps=1e-6).cpu()
    rows = sample_rows(m) if m == 816 else torch.arange(m)
    ar = a[rows].double()
    r = torch.rsqrt(ar.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = F.gelu((ar @ gq.t()) * r, approximate='tanh') * ((ar @ uq.t()) * r)
    assert rel_err(out[rows], ref) <= W16_TOL


def test_w8a16_wide_plain_and_qkv(K, cuda):
    """The wide kernel on PLAIN (M = 6528, 208 tiles) with bias and
    residual, sampled rows."""
    announce('w8a16 wide plain m=6528 n=2048 k=2048')
    m, n, k = 6528, 2048, 2048
    a = randn((m, k), 230, std=1.5)
    fw, wq = fp8_weight(K, randn((n, k), 231, std=0.02), cuda, act='bf16')
    bias = randn((n,), 232, std=0.5)
    res = randn((m, n), 233)
    out = K.gemm(a.to(cuda), fw, bias=bias.to(cuda), residual=res.to(cuda))
    rows = sample_rows(m)
    ref = a[rows].double() @ wq.t() + bias.double() + res[rows].double()
    assert rel_err(out.cpu()[rows], ref) <= W16_TOL


def test_w8a16_wide_split_k_down(K, cuda):
    """The bs=1 prefix down projection shape (M = 816, K = 16384): the wide
    kernel over 8 K ranges with the weight-scaled partials, then the reduce
    (residual in place, row sums of squares of the output)."""
    announce('w8a16 wide split-K down m=816 k=16384')
    m, n, k = 816, 2048, 16384
    a = randn((m, k), 240)
    fw, wq = fp8_weight(K, randn((n, k), 241, std=0.01), cuda, act='bf16')
    res = randn((m, n), 242)
    x = res.to(cuda)
    ss = torch.zeros(K.ss_parts(n), m, device=cuda)
    K.gemm(a.to(cuda), fw, out=x, residual=x, ss_out=ss)
    rows = sample_rows(m)
    got = x.cpu()
    ref = a[rows].double() @ wq.t() + res[rows].double()
    assert rel_err(got[rows], ref) <= W16_TOL
    want = got.double().view(m, -1, 64).pow(2).sum(-1).t()
    assert ((ss.cpu().double() - want).abs() <= 1e-5 * want + 1e-6).all()
