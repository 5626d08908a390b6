"""The decode attention's in-launch merge (the bs=1 expert shape: 51 tokens x
8 heads against 867 cached keys, 14 key ranges merged inside the launch).

* Every call leaves the 64 KiB counter region of the attention workspace at
  zero (arrival counts, merger counts and the status word).
* A merge whose bounded wait runs out is reported: the descriptor's test
  hook makes every merging workgroup give up at once (all kernels still run
  to their end), kernels.attention_check raises FvxError with status
  FVX_ERR_MERGE and clears the counters, and the next call is bitwise the
  result of a clean run.
"""
import pytest
import torch

from tests.conftest import announce

pytestmark = pytest.mark.gpu

COUNTER_BYTES = 64 * 1024


@pytest.fixture(scope='module')
def K():
    from fluxvla_amd import kernels
    return kernels


def _expert_case(cuda, seed):
    g = torch.Generator().manual_seed(seed)
    P, Ss, H, D, T = 816, 51, 8, 256, 872
    q = torch.randn(1, Ss, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, T, D, generator=g).to(torch.bfloat16)
    vt = torch.randn(1, D, T, generator=g).to(torch.bfloat16)
    cum = torch.cumsum(torch.tensor([1, 1] + [0] * 49), 0).to(torch.int32)
    kgrp = torch.cat([torch.zeros(P, dtype=torch.int32), cum])[None]
    qgrp = cum[None]
    return [t.to(cuda) for t in (q, k[:, :P + Ss], vt, kgrp, qgrp)]


def _run(K, cuda, case, **kw):
    q, k, vt, kgrp, qgrp = case
    o = torch.empty_like(q)
    K.mqa_attention(q, k, vt, o, kgrp, qgrp, v_transposed=True, **kw)
    return o


def test_counters_left_zero(K, cuda):
    announce('attention merge counters left zero')
    case = _expert_case(cuda, 1)
    outs = [_run(K, cuda, case) for _ in range(3)]
    torch.cuda.synchronize()
    ws = K.workspace(cuda, 'attn')
    assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0
    K.attention_check(cuda)          # no error
    assert all(torch.equal(o, outs[0]) for o in outs)


def test_wait_expiry_is_reported_and_cleared(K, cuda):
    from fluxvla_amd._lib import FVX_ERR_MERGE, FvxError
    announce('attention merge wait expiry')
    case = _expert_case(cuda, 2)
    clean = _run(K, cuda, case)
    K.attention_check(cuda)
    # the merging workgroups give up at once, on other inputs (so stale
    # partials cannot happen to equal the right ones)
    _run(K, cuda, _expert_case(cuda, 3), merge_no_wait=True)
    with pytest.raises(FvxError) as e:
        K.attention_check(cuda)
    assert e.value.code == FVX_ERR_MERGE
    assert 'stopped waiting' in str(e.value)
    ws = K.workspace(cuda, 'attn')
    assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0
    K.attention_check(cuda)          # cleared: no error left behind
    again = _run(K, cuda, case)
    K.attention_check(cuda)
    assert torch.equal(again, clean)


def test_fragment_only_output(K, cuda):
    """o_row_major=False (the bs=1 expert, whose o-projection reads the
    fragment-major copy): the fragment-major output equals the one written
    next to the row-major output, and the row-major buffer is untouched."""
    announce('attention fragment-only output')
    q, k, vt, kgrp, qgrp = _expert_case(cuda, 4)
    Ss, H, D = q.shape[1], q.shape[2], q.shape[3]
    both_o = torch.empty_like(q)
    f1 = K.FragA.empty(H * D, cuda).rows(Ss)
    f1.buf.zero_()
    K.mqa_attention(q, k, vt, both_o, kgrp, qgrp, v_transposed=True, o_frag=f1)
    only_o = torch.full_like(q, 7.0)
    f2 = K.FragA.empty(H * D, cuda).rows(Ss)
    f2.buf.zero_()
    K.mqa_attention(q, k, vt, only_o, kgrp, qgrp, v_transposed=True, o_frag=f2,
                    o_row_major=False)
    K.attention_check(cuda)
    assert torch.equal(f1.buf, f2.buf)
    assert bool((only_o == 7.0).all())
