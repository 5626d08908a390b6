"""The registered types driven through the reference runners' sequence on the
GPU (serve.py:45-66, libero_eval_runner.py:89-95, 170-181): Registry build
from the config dict -> load_state_dict(strict=True) -> eval -> to(device)
-> predict_action, checked against the CPU oracle (chunk max abs error
<= 2e-2).  Reduced depth (1 layer per tower) and vocab (1024) so the oracle
finishes in seconds."""
import pytest
import torch

from fluxvla_amd import registry as R
from fluxvla_amd.weights import make_inputs, make_state_dict
from oracle import pi0_oracle as O
from tests.conftest import announce
from tests.test_registry import StandInRegistry, reference_cfg

pytestmark = pytest.mark.gpu

CHUNK_ATOL = 2e-2


def _oracle(sd, cfg, inp):
    return O.predict_action(sd, cfg, inp['images'], inp['lang_tokens'],
                            inp['states'], inp['img_masks'],
                            inp['lang_masks'], inp['noise'])


def _predict(vla, inp, dev):
    return vla.predict_action(**{k: v.to(dev) for k, v in inp.items()})


@pytest.mark.parametrize('name,extra', [
    ('PI0FlowMatching', {}),
    ('PI05FlowMatchingInference', dict(num_views=3)),
    # the libero PI0.5 config: 2 views, 10-step chunk
    # (configs/pi05/pi05_paligemma_libero_10_full_inference.py:118-181)
    ('PI05FlowMatchingInference', dict(num_views=2, n_action_steps=10)),
])
def test_runner_sequence_matches_oracle(cuda, name, extra):
    announce(f'registry sequence {name} {extra}')
    reg = R.register_into(StandInRegistry())
    vla = reg.build(reference_cfg(name, layers=1, vocab=1024, vit_layers=1,
                                  **extra))
    cfg = vla.config
    sd = make_state_dict(cfg, seed=21)
    vla.load_state_dict(sd, strict=True)
    vla = vla.eval()
    vla.to(device=cuda.index, dtype=torch.bfloat16)
    assert vla.inference_model is None          # prepared lazily
    inp = make_inputs(cfg, batch=1, seed=22)
    got = _predict(vla, inp, cuda)
    assert vla.inference_model is not None
    assert got.shape == (1, cfg.n_action_steps, cfg.max_action_dim)
    assert got.dtype == torch.float32 and got.device == cuda
    err = (got.cpu() - _oracle(sd, cfg, inp)).abs().max().item()
    print(f'chunk max abs err {err:.3e}')
    assert err <= CHUNK_ATOL
    # a second call replays the prepared model
    m = vla.inference_model
    assert torch.equal(_predict(vla, inp, cuda), got)
    assert vla.inference_model is m


def test_new_weights_are_served_not_stale(cuda):
    """load_state_dict after a call drops the prepared model (and its
    captured graph): the next chunk follows the new weights."""
    announce('registry reload')
    vla = R.build_vla_from_cfg(reference_cfg('PI0FlowMatching', layers=1,
                                             vocab=1024, vit_layers=1))
    cfg = vla.config
    sd1 = make_state_dict(cfg, seed=31)
    sd2 = make_state_dict(cfg, seed=32)
    inp = make_inputs(cfg, batch=1, seed=33)
    vla.load_state_dict(sd1)
    vla.to(cuda)
    first = _predict(vla, inp, cuda)
    vla.load_state_dict(sd2)
    second = _predict(vla, inp, cuda).cpu()
    err = (second - _oracle(sd2, cfg, inp)).abs().max().item()
    assert err <= CHUNK_ATOL
    assert (second - first.cpu()).abs().max().item() > 10 * CHUNK_ATOL


def test_eager_type_takes_prompt_length_from_the_request(cuda):
    """PI0FlowMatching takes the prompt length from the request (48 by
    default); a longer prompt prepares a longer buffer, padded prompts
    (ProcessPrompts pads past the last token) do not."""
    announce('registry prompt length')
    vla = R.build_vla_from_cfg(reference_cfg('PI0FlowMatching', layers=1,
                                             vocab=1024, vit_layers=1))
    sd = make_state_dict(vla.config, seed=41)
    vla.load_state_dict(sd)
    vla.to(cuda)
    inp = make_inputs(vla.config.scaled(max_prompt_len=60), batch=1, seed=42)
    got = _predict(vla, inp, cuda)
    assert vla.inference_model.cfg.max_prompt_len == 64
    cfg = vla.inference_model.cfg
    err = (got.cpu() - _oracle(sd, cfg, inp)).abs().max().item()
    assert err <= CHUNK_ATOL
    # 180 tokens of which 20 are valid: the prepared 64-token buffer serves
    m = vla.inference_model
    ids = torch.zeros(1, 180, dtype=torch.long)
    ids[:, :20] = inp['lang_tokens'][:, :20]
    mask = torch.zeros(1, 180, dtype=torch.bool)
    mask[:, :20] = True
    short = dict(inp, lang_tokens=ids, lang_masks=mask)
    got = _predict(vla, short, cuda)
    assert vla.inference_model is m
    ref_inp = dict(inp, lang_tokens=ids[:, :20], lang_masks=mask[:, :20])
    err = (got.cpu() - _oracle(sd, cfg, ref_inp)).abs().max().item()
    assert err <= CHUNK_ATOL
