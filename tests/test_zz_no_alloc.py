"""fvx_gemm_noalloc (split-K scratch in the library's static device array)
against fvx_gemm with a caller-passed workspace, through the C ABI: the
same kernels must give bitwise the same output.  Two calls in a row, the
second with a smaller input, on the split-K paths that use the scratch
(skinny M <= 64 with K ranges; M > 64 over K ranges with the reduce
pass); a problem whose scratch need exceeds the static array is refused
without a launch."""
import ctypes

import pytest
import torch

from fluxvla_amd import _lib
from fluxvla_amd import kernels as K
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _operands(m, n, k, seed, dev):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(m, k, generator=g).bfloat16().to(dev)
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16().to(dev)
    b = (torch.randn(n, generator=g) * 0.1).bfloat16().to(dev)
    r = torch.randn(m, n, generator=g).bfloat16().to(dev)
    return a, w, b, r


@pytest.mark.parametrize('shape', [
    # (m, n, k), then the smaller second call
    ((51, 1024, 8192), (20, 1024, 8192)),     # skinny, 4 K ranges
    ((300, 512, 8192), (272, 512, 8192)),     # wide kernel, 8 K ranges + reduce
])
def test_noalloc_matches_workspace_gemm(cuda, shape):
    for i, (m, n, k) in enumerate(shape):
        announce(f'gemm_noalloc call {i} m={m} n={n} k={k}')
        a, w, b, r = _operands(m, n, k, seed=60 + i, dev=cuda)
        d = K._gemm_desc(a, w)
        assert K.fvx_workspace_bytes(d) > 0, 'case must use the scratch'
        want = K.gemm(a, w, bias=b, residual=r)
        got = K.gemm(a, w, bias=b, residual=r, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        ref = a.float() @ w.float().t() + b.float() + r.float()
        err = ((got.float() - ref).abs().max() / ref.abs().max()).item()
        assert err <= 1e-2


def test_noalloc_refuses_oversized_scratch(cuda):
    """Prefix down projection at bs=1 (8 K ranges of fp32 partials, ~53 MB)
    exceeds the 32 MiB static scratch: refused, nothing launched."""
    announce('gemm_noalloc oversized refusal')
    m, n, k = 816, 2048, 16384
    a = torch.zeros(m, k, dtype=torch.bfloat16, device=cuda)
    w = torch.zeros(n, k, dtype=torch.bfloat16, device=cuda)
    d = K._gemm_desc(a, w)
    assert K.fvx_workspace_bytes(d) > _lib.GEMM_NOALLOC_SCRATCH_BYTES
    out = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(_lib.FvxError) as e:
        K.gemm(a, w, out=out, noalloc=True)
    assert e.value.code == _lib.FVX_ERR_WORKSPACE
    assert 'static scratch' in str(e.value)
    torch.cuda.synchronize()
    assert (out == 7.0).all()
