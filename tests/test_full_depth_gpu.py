"""The full configurations against the CPU oracle at bs=1: PI0 and PI0.5 at
their real depth (SigLIP 27 layers, Gemma-2B 18, action expert 18), the
257,152-token vocabulary, the 816-token prefix and 10 Euler steps -- what
the reduced-depth tests of test_pi0_gpu.py leave out.  Bar from the north
star: the 50 x 32 action chunk within max abs error 2e-2 of the fp32
oracle (pi0_flowmatching.py:702-831 / pi05_flowmatching.py restated)."""
import os

import pytest
import torch

from fluxvla_amd.config import PI0, PI05
from fluxvla_amd.weights import make_inputs, make_state_dict
from oracle import pi0_oracle as O
from tests.conftest import announce

pytestmark = pytest.mark.gpu

CHUNK_ATOL = 2e-2


@pytest.mark.parametrize('pi05', [False, True])
def test_full_depth_chunk_matches_oracle(cuda, pi05):
    from fluxvla_amd.pi0_inference import PI0Inference
    cfg = PI05 if pi05 else PI0
    announce(f'full-depth chunk pi05={pi05}')
    sd = make_state_dict(cfg, seed=5, device=cuda)
    inp = make_inputs(cfg, batch=1, seed=6)
    m = PI0Inference(cfg, sd, device=cuda, max_batch=1)
    got = m.predict_action(inp['images'].to(cuda), inp['lang_tokens'].to(cuda),
                           inp['states'].to(cuda), inp['img_masks'].to(cuda),
                           inp['lang_masks'].to(cuda), noise=inp['noise'].to(cuda)).cpu()
    del m
    sdc = {k: v.cpu() for k, v in sd.items()}
    del sd
    torch.cuda.empty_cache()
    torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))
    ref = O.predict_action(sdc, cfg, inp['images'], inp['lang_tokens'], inp['states'],
                           inp['img_masks'], inp['lang_masks'], inp['noise'])
    err = (got - ref).abs().max().item()
    print(f'full-depth chunk max abs err {err:.3e} (|ref| max {ref.abs().max():.2f})')
    assert err <= CHUNK_ATOL


@pytest.mark.parametrize('pi05', [False, True])
def test_full_depth_guidance_vjp_chunk_matches_oracle(cuda, pi05):
    """Guidance RTC with use_vjp at the full depth: the backward pass through
    all 18 expert layers against the oracle's torch autograd."""
    from fluxvla_amd.pi0_inference import PI0Inference
    cfg = PI05 if pi05 else PI0
    announce(f'full-depth guidance-vjp chunk pi05={pi05}')
    sd = make_state_dict(cfg, seed=7, device=cuda)
    inp = make_inputs(cfg, batch=1, seed=8)
    prev = torch.randn(1, 40, cfg.max_action_dim,
                       generator=torch.Generator().manual_seed(9)) * 0.5
    rc = {'enabled': True, 'method': 'guidance', 'use_vjp': True,
          'max_guidance_weight': 5.0, 'decay_end': 20}
    m = PI0Inference(cfg, sd, device=cuda, max_batch=1)
    got = m.predict_action(inp['images'].to(cuda), inp['lang_tokens'].to(cuda),
                           inp['states'].to(cuda), inp['img_masks'].to(cuda),
                           inp['lang_masks'].to(cuda), noise=inp['noise'].to(cuda),
                           prev_actions=prev.to(cuda), prefix_len=6,
                           rtc_config=rc).cpu()
    del m
    sdc = {k: v.cpu() for k, v in sd.items()}
    del sd
    torch.cuda.empty_cache()
    torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))
    ref = O.predict_action(sdc, cfg, inp['images'], inp['lang_tokens'], inp['states'],
                           inp['img_masks'], inp['lang_masks'], inp['noise'],
                           prev_actions=prev, prefix_len=6, rtc_config=rc)
    err = (got - ref).abs().max().item()
    print(f'full-depth guidance-vjp chunk max abs err {err:.3e} '
          f'(|ref| max {ref.abs().max():.2f})')
    assert err <= CHUNK_ATOL
