"""The adaptive RMSNorm folded into the M <= 64 GEMMs (fvx_gemm_desc.a_scale
with the QKV_ROPE / GEGLU fp32 biases), against an fp32 restatement of
GemmaRMSNorm's adaptive mode followed by the GEMM (condition_gemma.py:
126-145): y = rms(x) * (1 + scale) + shift, then y @ W^T.  bf16 and W8A16
weights.  Bar: rel <= 1e-2 (the reference rounds y to bf16; the fold rounds
x * (1 + scale) instead)."""
import pytest
import torch
import torch.nn.functional as F

from tests.conftest import announce

pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(shape, seed, std=1.0):
    return (torch.randn(shape, generator=gen(seed)) * std).to(torch.bfloat16)


def rel_err(out, ref):
    out, ref = out.detach().float().cpu(), ref.detach().float().cpu()
    return ((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


@pytest.fixture(scope='module')
def K():
    from fluxvla_amd import kernels
    kernels._lib.load()
    return kernels


def ada_ref(x, scale, shift, eps=1e-6):
    xf = x.float()
    n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return n * (1 + scale.float()) + shift.float()


@pytest.mark.parametrize('fp8', [False, True])
@pytest.mark.parametrize('m', [50, 17])
def test_folded_geglu(K, cuda, fp8, m):
    announce(f'folded adarms geglu m={m} fp8={fp8}')
    x = randn((m, 1024), 1, std=3.0)
    sc, sh = randn((1024,), 2, std=0.3), randn((1024,), 3, std=0.3)
    wg, wu = randn((4096, 1024), 4, std=0.02), randn((4096, 1024), 5, std=0.02)
    if fp8:
        g8 = K.Fp8Weight.quantize(wg.to(cuda)).pack_frag()
        u8 = K.Fp8Weight.quantize(wu.to(cuda)).pack_frag()
        wg_eff = K.Fp8Weight.quantize(wg.to(cuda)).dequantize().cpu()
        wu_eff = K.Fp8Weight.quantize(wu.to(cuda)).dequantize().cpu()
        gw, uw = g8, u8
    else:
        gw, uw = K.FragB.pack(wg.to(cuda)), K.FragB.pack(wu.to(cuda))
        wg_eff, wu_eff = wg.float(), wu.float()
    bg = (sh.float() @ wg_eff.t()).to(cuda)
    bu = (sh.float() @ wu_eff.t()).to(cuda)
    xf = K.FragA.empty(1024, cuda).rows(m)
    K.pack_frag(x.to(cuda), xf)
    out = torch.empty(m, 4096, dtype=torch.bfloat16, device=cuda)
    K.gemm_geglu(xf, gw, uw, out=out, rownorm_eps=1e-6, a_scale=sc.to(cuda),
                 bias_f32=bg, bias2_f32=bu)
    y = ada_ref(x, sc, sh)
    ref = F.gelu(y @ wg_eff.t(), approximate='tanh') * (y @ wu_eff.t())
    assert rel_err(out, ref) <= 1e-2


def test_folded_qkv_matches_norm_then_qkv(K, cuda):
    """Q|K|V + RoPE from the folded GEMM against the adaRMS kernel followed
    by the plain QKV GEMM (both checked elsewhere against fp32 references)."""
    announce('folded adarms qkv+rope m=50')
    m, hd = 50, 256
    x = randn((m, 1024), 11, std=2.0)
    sc, sh = randn((1024,), 12, std=0.3), randn((1024,), 13, std=0.3)
    w = randn((10 * hd, 1024), 14, std=0.02).to(cuda)
    wf = K.FragB.pack(w)
    rope = K.rope_table(1024, hd, 10000.0, device=cuda)
    pos = torch.arange(800, 800 + m, dtype=torch.int32, device=cuda)
    outs = []
    for fold in (False, True):
        q = torch.zeros(m, 8 * hd, dtype=torch.bfloat16, device=cuda)
        k = torch.zeros(m, hd, dtype=torch.bfloat16, device=cuda)
        v = torch.zeros(m, hd, dtype=torch.bfloat16, device=cuda)
        if fold:
            xf = K.FragA.empty(1024, cuda).rows(m)
            K.pack_frag(x.to(cuda), xf)
            bias = (sh.float().to(cuda)[None] @ w.float().t())[0].contiguous()
            K.gemm_qkv_rope(xf, wf, rope, pos, q, k, v, 8, hd, rownorm_eps=1e-6,
                            a_scale=sc.to(cuda), bias_f32=bias)
        else:
            style = torch.cat([sc, sh, torch.zeros(1024, dtype=torch.bfloat16)])
            xn = torch.empty(m, 1024, dtype=torch.bfloat16, device=cuda)
            K.adarms_norm(x.to(cuda), style[None].to(cuda), out=xn, eps=1e-6)
            K.gemm_qkv_rope(xn, wf, rope, pos, q, k, v, 8, hd)
        outs.append((q.cpu(), k.cpu(), v.cpu()))
    for a, b in zip(*outs):
        assert rel_err(b, a) <= 1e-2


def test_folded_euler(K, cuda):
    announce('folded adarms euler m=50')
    m = 50
    x = randn((m, 1024), 21, std=2.0)
    sc, sh = randn((1024,), 22, std=0.3), randn((1024,), 23, std=0.3)
    w = randn((32, 1024), 24, std=0.02)
    b = randn((32,), 25, std=0.1)
    xt0 = torch.randn(m, 32, generator=gen(26))
    xt = xt0.clone().to(cuda)
    bias = (sh.float() @ w.float().t()).to(cuda)
    K.gemm_euler(x.to(cuda), w.to(cuda), b.to(cuda), xt, -0.1, rownorm_eps=1e-6,
                 bias_f32=bias, a_scale=sc.to(cuda))
    v = ada_ref(x, sc, sh) @ w.float().t() + b.float()
    assert (xt.cpu() - (xt0 - 0.1 * v)).abs().max().item() <= 2e-3


def test_fold_refusals(K, cuda):
    """a_scale only on M <= 64 QKV / GEGLU / EULER GEMMs; no bf16 bias and no
    fp32 bias without it on QKV / GEGLU."""
    a = randn((100, 1024), 31).to(cuda)
    w = randn((512, 1024), 32, std=0.02).to(cuda)
    with pytest.raises(ValueError):
        K.gemm_geglu(a, w, w, a_scale=torch.zeros(1024, dtype=torch.bfloat16,
                                                  device=cuda))
    with pytest.raises(ValueError):
        K.gemm_geglu(a[:50], w, w, bias_f32=torch.zeros(512, device=cuda))
