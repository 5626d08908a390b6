"""Real-time chunking (RTC) on the GPU: the Euler / suffix-embedding GEMM and
adaRMS epilogues that carry it, against fp32 references of the same op, and
whole chunks (PI0, PI0.5; prefix and guidance methods) against the CPU
oracle's restatement of PI0FlowMatching._predict_action_prefix_rtc /
_predict_action_guidance_rtc (fluxvla/models/vlas/pi0_flowmatching.py:
651-700) and rtc_guidance.py:28-155 (use_vjp by torch autograd).

Bars as for the plain chunk: max abs error 2e-2 on the 50 x 32 chunk; the
locked prefix rows are exactly the previous chunk; kernel outputs within
2e-3 absolute of the fp32 Euler reference (rel 1e-2 for bf16 outputs).
"""
import pytest
import torch

from fluxvla_amd.config import tiny
from fluxvla_amd.weights import make_inputs, make_state_dict
from oracle import pi0_oracle as O
from tests.conftest import announce

pytestmark = pytest.mark.gpu

CHUNK_ATOL = 2e-2


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


# ---------------------------------------------------------------------------
# Kernels
# ---------------------------------------------------------------------------
@pytest.mark.parametrize('m,lock', [(50, 7), (50, 0), (50, 50), (100, 13)])
def test_euler_prefix_lock(K, cuda, m, lock):
    """Locked rows (m % 50 < lock) store the previous chunk; the others take
    the plain Euler update.  m = 100: two chunks in one GEMM (tile path)."""
    announce(f'gemm euler rtc prefix m={m} lock={lock}')
    x = randn((m, 1024), 1, std=2.0)
    w = randn((32, 1024), 2, std=0.02)
    b = randn((32,), 3, std=0.1)
    xt0 = torch.randn(m, 32, generator=gen(4))
    prev = torch.randn(m, 32, generator=gen(5))
    xt = xt0.clone().to(cuda)
    xtb = torch.empty(m, 32, dtype=torch.bfloat16, device=cuda)
    lk = torch.tensor([lock], dtype=torch.int32, device=cuda)
    K.gemm_euler(x.to(cuda), w.to(cuda), b.to(cuda), xt, -0.1, xt_bf16=xtb,
                 rownorm_eps=1e-6, rtc_lock=lk, rtc_period=50,
                 rtc_prev=prev.to(cuda))
    xf = x.float()
    v = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
         @ w.float().t() + b.float())
    ref = xt0 - 0.1 * v
    locked = (torch.arange(m) % 50) < lock
    ref[locked] = prev[locked]
    got = xt.cpu()
    assert torch.equal(got[locked], prev[locked])
    assert (got - ref).abs().max().item() <= 2e-3
    assert torch.equal(xtb.cpu(), got.bfloat16())


@pytest.mark.parametrize('m', [50, 100])
def test_euler_guidance(K, cuda, m):
    """x + dt v + cw[r] (prev - x + omt v), r = m % 50, cw 0 past row 40."""
    announce(f'gemm euler rtc guidance m={m}')
    x = randn((m, 1024), 11, std=2.0)
    w = randn((32, 1024), 12, std=0.02)
    b = randn((32,), 13, std=0.1)
    xt0 = torch.randn(m, 32, generator=gen(14))
    prev = torch.randn(m, 32, generator=gen(15))
    cw = torch.rand(50, generator=gen(16)) * 0.5
    cw[40:] = 0.0
    omt = 0.7
    xt = xt0.clone().to(cuda)
    K.gemm_euler(x.to(cuda), w.to(cuda), b.to(cuda), xt, -0.1,
                 rownorm_eps=1e-6, rtc_period=50, rtc_prev=prev.to(cuda),
                 rtc_cw=cw.to(cuda), rtc_omt=omt)
    xf = x.float()
    v = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
         @ w.float().t() + b.float())
    c = cw[torch.arange(m) % 50][:, None]
    ref = xt0 - 0.1 * v + c * (prev - xt0 + omt * v)
    assert (xt.cpu() - ref).abs().max().item() <= 2e-3


@pytest.mark.parametrize('m', [50, 100])
def test_plain_bias_f32_locked(K, cuda, m):
    """Suffix-embedding GEMM: locked rows add the time-0 bias row."""
    announce(f'gemm plain bias_f32_locked m={m}')
    a = randn((m, 1024), 21)
    w = randn((1024, 1024), 22, std=0.02)
    bias = torch.randn(1024, generator=gen(23))
    bias0 = torch.randn(1024, generator=gen(24))
    lk = torch.tensor([9], dtype=torch.int32, device=cuda)
    out = K.gemm(a.to(cuda), w.to(cuda), bias_f32=bias.to(cuda),
                 bias_f32_locked=bias0.to(cuda), rtc_lock=lk, rtc_period=50,
                 act=K._lib.ACT_SILU)
    locked = ((torch.arange(m) % 50) < 9)[:, None]
    ref = torch.nn.functional.silu(a.float() @ w.float().t() +
                                   torch.where(locked, bias0, bias))
    assert rel_err(out, ref) <= 1e-2


def test_adarms_norm_locked(K, cuda):
    """Rows with row % 50 < lock take the locked style row (scale, shift
    and gate)."""
    announce('adarms_norm_locked [100,1024]')
    x = randn((100, 1024), 31)
    style = randn((1, 3072), 32, std=0.2)
    style0 = randn((3072,), 33, std=0.2)
    lk = torch.tensor([6], dtype=torch.int32, device=cuda)
    y = torch.empty(100, 1024, dtype=torch.bfloat16, device=cuda)
    gt = torch.empty_like(y)
    K.adarms_norm(x.to(cuda), style.to(cuda), y, gt, style_locked=style0.to(cuda),
                  lock=lk, lock_period=50)
    locked = ((torch.arange(100) % 50) < 6)[:, None]
    st = torch.where(locked, style0.float()[None], style.float())
    xf = x.float()
    n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = n * (1 + st[:, :1024]) + st[:, 1024:2048]
    assert rel_err(y, ref) <= 1e-2
    assert torch.equal(gt.cpu(), st[:, 2048:].bfloat16())


# ---------------------------------------------------------------------------
# Whole chunks against the oracle
# ---------------------------------------------------------------------------
@pytest.fixture(scope='module')
def models():
    from fluxvla_amd.pi0_inference import PI0Inference
    cache = {}

    def get(pi05):
        if pi05 not in cache:
            # 14 real action dims: the previous chunk is zero-padded to 32
            cfg = tiny(pi05=pi05, ori_action_dim=14)
            sd = make_state_dict(cfg, seed=40)
            m = PI0Inference(cfg, sd, device='cuda', max_batch=2)
            cache[pi05] = (cfg, sd, m)
        return cache[pi05]

    return get


def _oracle(cfg, sd, inp, prev, prefix_len, rtc_config, kvs=None):
    """The oracle's RTC loop over a prefix cache computed once per input."""
    states = inp['states'].float()
    if kvs is None:
        kvs = O.prefix_forward(sd, cfg, inp['images'], inp['lang_tokens'],
                               inp['img_masks'], inp['lang_masks'])
    cache, pad = kvs
    prev, method = O.rtc_inputs(cfg, prev, prefix_len, rtc_config)
    dt = torch.tensor(-1.0 / cfg.num_steps, dtype=torch.float32)
    x = inp['noise'].float().clone()
    B = x.shape[0]

    def denoise(xx, t):
        return O.denoise_step(sd, cfg, states, pad, cache, xx, t)

    if method == 'prefix':
        out = O.euler_prefix_rtc(x, denoise, B, dt, prev, prefix_len,
                                 cfg.n_action_steps)
    else:
        out = O.euler_guidance_rtc(x, denoise, B, dt, prev, prefix_len,
                                   rtc_config, cfg.n_action_steps)
    return out, kvs


def _run(m, inp, cuda, prev, prefix_len, rtc_config):
    return m.predict_action(inp['images'].to(cuda), inp['lang_tokens'].to(cuda),
                            inp['states'].to(cuda), inp['img_masks'].to(cuda),
                            inp['lang_masks'].to(cuda),
                            noise=inp['noise'].to(cuda),
                            prev_actions=prev.to(cuda), prefix_len=prefix_len,
                            rtc_config=rtc_config).cpu()


@pytest.mark.parametrize('pi05', [False, True])
@pytest.mark.parametrize('batch', [1, 2])
def test_prefix_rtc_chunk(models, cuda, pi05, batch):
    """Prefix method at two prefix lengths through one captured graph; the
    locked rows are exactly the previous chunk."""
    cfg, sd, m = models(pi05)
    inp = make_inputs(cfg, batch=batch, seed=41)
    prev = torch.randn(batch, 30, 14, generator=gen(42)) * 0.5
    kvs = None
    for p in (8, 3):
        announce(f'pi0 prefix-rtc chunk pi05={pi05} batch={batch} prefix={p}')
        rc = {'enabled': True, 'method': 'prefix'}
        ref, kvs = _oracle(cfg, sd, inp, prev, p, rc, kvs)
        got = _run(m, inp, cuda, prev, p, rc)
        err = (got - ref).abs().max().item()
        print(f'prefix {p}: chunk max abs err {err:.3e}')
        assert err <= CHUNK_ATOL
        assert torch.equal(got[:, :p, :14], prev[:, :p])
        assert got[:, :p, 14:].abs().max().item() == 0.0


@pytest.mark.parametrize('pi05', [False, True])
@pytest.mark.parametrize('schedule', ['exp', 'linear'])
def test_guidance_rtc_chunk(models, cuda, pi05, schedule):
    """Guidance method (no VJP) with a previous chunk shorter than the new
    one: rows past it are unguided."""
    announce(f'pi0 guidance-rtc chunk pi05={pi05} schedule={schedule}')
    cfg, sd, m = models(pi05)
    inp = make_inputs(cfg, batch=1, seed=43)
    prev = torch.randn(1, 40, 14, generator=gen(44)) * 0.5
    rc = {'enabled': True, 'method': 'guidance', 'schedule': schedule,
          'max_guidance_weight': 5.0, 'decay_end': 20}
    ref, _ = _oracle(cfg, sd, inp, prev, 6, rc)
    got = _run(m, inp, cuda, prev, 6, rc)
    err = (got - ref).abs().max().item()
    print(f'chunk max abs err {err:.3e}')
    assert err <= CHUNK_ATOL
    # the plain chunk (same request) differs: the guidance acted
    plain = m.predict_action(inp['images'].to(cuda), inp['lang_tokens'].to(cuda),
                             inp['states'].to(cuda), noise=inp['noise'].to(cuda)).cpu()
    assert (plain - got).abs().max().item() > 10 * CHUNK_ATOL


def test_rtc_falls_back_to_plain(models, cuda):
    """prefix_len 0, no rtc_config or an unknown method: the plain loop
    (pi0_flowmatching.py:753-785), bitwise the same chunk."""
    announce('pi0 rtc fallbacks')
    cfg, sd, m = models(False)
    inp = make_inputs(cfg, batch=1, seed=45)
    prev = torch.randn(1, 30, 14, generator=gen(46))
    plain = m.predict_action(inp['images'].to(cuda), inp['lang_tokens'].to(cuda),
                             inp['states'].to(cuda), noise=inp['noise'].to(cuda)).cpu()
    for p, rc in ((0, {'method': 'prefix'}), (5, None), (5, {'method': 'other'}),
                  (0, {'method': 'guidance', 'use_vjp': True})):
        got = _run(m, inp, cuda, prev, p, rc)
        assert torch.equal(got, plain)


@pytest.mark.parametrize('pi05', [False, True])
@pytest.mark.parametrize('batch', [1, 2])
def test_guidance_vjp_rtc_chunk(models, cuda, pi05, batch):
    """Guidance with use_vjp (rtc_guidance.py:142-150): the correction
    pulled back through the expert's Jacobian by the backward kernels,
    against the oracle's torch-autograd loop.  The VJP term moves the chunk
    by far more than the bar (the oracle with and without it), so a product
    that dropped or mis-signed it would fail."""
    announce(f'pi0 guidance-vjp chunk pi05={pi05} batch={batch}')
    cfg, sd, m = models(pi05)
    inp = make_inputs(cfg, batch=batch, seed=47)
    prev = torch.randn(batch, 40, 14, generator=gen(48)) * 0.5
    rc = {'enabled': True, 'method': 'guidance', 'use_vjp': True,
          'schedule': 'exp', 'max_guidance_weight': 5.0, 'decay_end': 20}
    ref, kvs = _oracle(cfg, sd, inp, prev, 6, rc)
    plain_ref, _ = _oracle(cfg, sd, inp, prev, 6, dict(rc, use_vjp=False), kvs)
    got = _run(m, inp, cuda, prev, 6, rc)
    plain = _run(m, inp, cuda, prev, 6, dict(rc, use_vjp=False))
    err = (got - ref).abs().max().item()
    moved, moved_got = ref - plain_ref, got - plain
    d_err = (moved_got - moved).abs().max().item()
    print(f'chunk max abs err {err:.3e}; the VJP term moves the chunk by '
          f'{moved.abs().max().item():.3e} (oracle), its move is off by '
          f'{d_err:.3e}')
    assert err <= CHUNK_ATOL
    # the VJP term's own effect (with minus without it) matches the
    # oracle's; dropping it would miss by the whole move (> 3e-2 here)
    assert moved.abs().max().item() > 3 * 0.5 * CHUNK_ATOL
    assert d_err <= 0.5 * CHUNK_ATOL
    # eager run of the same loop gives the graph's chunk
    m.use_graph = False
    try:
        eager = _run(m, inp, cuda, prev, 6, rc)
    finally:
        m.use_graph = True
    assert torch.equal(eager, got)


@pytest.mark.parametrize('pi05', [False, True])
@pytest.mark.parametrize('batch', [1, 2])
def test_guidance_vjp_step_matches_autograd(models, cuda, pi05, batch):
    """One VJP step on its own: after a chunk has filled the prefix cache,
    the step's forward (u) and backward (g = J_u^T e) at a chosen x_t against
    the oracle's denoise_step and torch autograd through it at the same
    bf16 input, with e = w (prev - x + (1 - t) u) as the product forms it."""
    announce(f'pi0 guidance-vjp one step pi05={pi05} batch={batch}')
    cfg, sd, m = models(pi05)
    inp = make_inputs(cfg, batch=batch, seed=49)
    prev = torch.randn(batch, 40, 14, generator=gen(50)) * 0.5
    rc = {'enabled': True, 'method': 'guidance', 'use_vjp': True,
          'max_guidance_weight': 5.0, 'decay_end': 25}
    m.use_graph = False
    try:
        _run(m, inp, cuda, prev, 8, rc)
    finally:
        m.use_graph = True
    eng, b = m._vjp, m._bufs[batch]
    na = cfg.n_action_steps
    x = torch.randn(batch, na, cfg.max_action_dim, generator=gen(51))
    b['xt'].copy_(x)
    b['xt_bf16'].copy_(x)
    step = 3
    eng.forward(b, batch, step)
    eng.backward(b, batch, step)
    v = eng.buffers(batch)
    u = v['u'].view(batch, na, -1).cpu()
    g = v['g'].view(batch, na, -1).cpu()
    cache, pad = O.prefix_forward(sd, cfg, inp['images'], inp['lang_tokens'],
                                  inp['img_masks'], inp['lang_masks'])
    xb = x.bfloat16().float()
    time = torch.tensor(m.times[step])
    with torch.enable_grad():
        xg = xb.clone().requires_grad_(True)
        u_ref = O.denoise_step(sd, cfg, inp['states'].float(), pad, cache, xg,
                               time.expand(batch))
        w = b['rtc_w'].cpu()
        prev_p = b['rtc_prev'].cpu()
        e = w[None, :, None] * (prev_p - x + m._rtc_omt[step] * u_ref.detach())
        (g_ref,) = torch.autograd.grad(u_ref, xg, e)
    eu, eg = rel_err(u, u_ref), rel_err(g, g_ref)
    cos = torch.nn.functional.cosine_similarity(g.flatten(), g_ref.flatten(),
                                                dim=0).item()
    print(f'u rel err {eu:.3e}; g rel err {eg:.3e}, cosine {cos:.5f}')
    assert eu <= 2e-2
    assert eg <= 5e-2 and cos >= 0.995


@pytest.mark.parametrize('weight_dtype', ['fp8', 'fp8_w8a8'])
def test_guidance_vjp_fp8_chunk(cuda, weight_dtype):
    """Guidance with use_vjp on fp8 weights (PI0.5, config 5): the backward
    runs on the dequantized weights, the forward on the fp8 GEMMs; against
    the oracle's VJP loop on the dequantized state dict, bs 1 and 2, within
    the bar of the plain fp8 chunk (2e-2 W8A16, 5e-2 W8A8)."""
    from fluxvla_amd.pi0_inference import PI0Inference
    cfg = tiny(pi05=True, ori_action_dim=14)
    sd = make_state_dict(cfg, seed=60)
    m = PI0Inference(cfg, sd, device='cuda', max_batch=2,
                     weight_dtype=weight_dtype)
    sdq = m.dequantized_state_dict(sd)
    bar = CHUNK_ATOL if weight_dtype == 'fp8' else 5e-2
    rc = {'enabled': True, 'method': 'guidance', 'use_vjp': True,
          'max_guidance_weight': 5.0, 'decay_end': 20}
    for batch in (1, 2):
        announce(f'guidance-vjp {weight_dtype} chunk batch={batch}')
        inp = make_inputs(cfg, batch=batch, seed=61)
        prev = torch.randn(batch, 40, 14, generator=gen(62)) * 0.5
        ref, _ = _oracle(cfg, sdq, inp, prev, 6, rc)
        got = _run(m, inp, cuda, prev, 6, rc)
        err = (got - ref).abs().max().item()
        print(f'{weight_dtype} guidance-vjp chunk max abs err {err:.3e}')
        assert err <= bar
