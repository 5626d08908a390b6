"""Weight ingestion end to end on the GPU: a checkpoint written in the
reference's on-disk names and read back through the PI0 name_mapping gives
bitwise the chunk of the in-memory state dict; an fp8 model built from the
quantization cache gives bitwise the chunk of one that quantized in memory
(real widths, one layer per tower)."""
import pytest
import torch

from fluxvla_amd import checkpoint as C
from fluxvla_amd.config import tiny
from fluxvla_amd.weights import make_inputs, make_state_dict
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _chunk(m, inp, cuda):
    return m.predict_action(inp['images'].to(cuda), inp['lang_tokens'].to(cuda),
                            inp['states'].to(cuda), inp['img_masks'].to(cuda),
                            inp['lang_masks'].to(cuda),
                            noise=inp['noise'].to(cuda)).cpu()


def test_from_pretrained_chunk_bitwise(cuda, tmp_path):
    from fluxvla_amd.pi0_inference import PI0Inference
    announce('checkpoint round trip chunk')
    cfg = tiny(vit_layers=1, llm_layers=1, exp_layers=1)
    sd = make_state_dict(cfg, seed=80)
    path = str(tmp_path / 'model.safetensors')
    C.export_checkpoint(sd, path)
    loaded = C.from_pretrained(cfg, path)
    inp = make_inputs(cfg, batch=1, seed=81)
    a = _chunk(PI0Inference(cfg, sd, device='cuda'), inp, cuda)
    b = _chunk(PI0Inference(cfg, loaded, device='cuda'), inp, cuda)
    assert torch.equal(a, b)


@pytest.mark.parametrize('weight_dtype', ['fp8', 'fp8_w8a8'])
def test_fp8_cache_chunk_bitwise(cuda, tmp_path, weight_dtype):
    from fluxvla_amd.pi0_inference import PI0Inference
    announce(f'fp8 cache chunk {weight_dtype}')
    cfg = tiny(pi05=True, vit_layers=1, llm_layers=1, exp_layers=1)
    sd = make_state_dict(cfg, seed=82)
    path = str(tmp_path / 'fp8.safetensors')
    inp = make_inputs(cfg, batch=1, seed=83)
    first = PI0Inference(cfg, sd, device='cuda', weight_dtype=weight_dtype,
                         fp8_cache=path)
    assert not first.fp8_cache_hit
    second = PI0Inference(cfg, sd, device='cuda', weight_dtype=weight_dtype,
                          fp8_cache=path)
    assert second.fp8_cache_hit
    for L1, L2 in zip(first.exp['layers'], second.exp['layers']):
        assert torch.equal(L1['qkv_w'].data, L2['qkv_w'].data)
        assert torch.equal(L1['down_w'].scale, L2['down_w'].scale)
    assert torch.equal(_chunk(first, inp, cuda), _chunk(second, inp, cuda))
    # other weights: the cache does not match and is rebuilt
    sd2 = dict(sd)
    k = 'llm_backbone.layers.0.mlp.down_proj.weight'
    sd2[k] = sd[k] * 2
    third = PI0Inference(cfg, sd2, device='cuda', weight_dtype=weight_dtype,
                         fp8_cache=path)
    assert not third.fp8_cache_hit
