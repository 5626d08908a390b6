"""Weight ingestion on the host: the reference's name_mapping rule
(base_vla.py:190-288) over safetensors files, shard directories and .pt
files, its error cases, and the fp8 cache's source hash.  The checkpoints
are written by tests/golden/make_tiny_checkpoint.py in the reference's
on-disk names."""
import os

import pytest
import torch
from safetensors.torch import load_file, save_file

from fluxvla_amd import checkpoint as C
from fluxvla_amd.weights import param_specs
from tests.golden import make_tiny_checkpoint as mk


@pytest.fixture(scope='module')
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp('ckpt')
    path = str(d / 'model.safetensors')
    cfg, sd = mk.write(path)
    return cfg, sd, path


def test_export_uses_reference_names(ckpt):
    cfg, sd, path = ckpt
    raw = load_file(path)
    assert len(raw) == len(sd)
    for k in ('paligemma_with_expert.gemma_expert.model.layers.0.mlp.down_proj.weight',
              'paligemma_with_expert.paligemma.model.language_model.layers.0.'
              'self_attn.q_proj.weight',
              'paligemma_with_expert.paligemma.model.vision_tower.vision_model.'
              'embeddings.patch_embedding.weight',
              'paligemma_with_expert.paligemma.model.multi_modal_projector.linear.weight',
              'action_time_mlp_in.weight', 'state_proj.bias'):
        assert k in raw, k
    assert not any(k.startswith('llm_backbone.') for k in raw)


def test_from_pretrained_roundtrip_file_dir_and_pt(ckpt, tmp_path):
    cfg, sd, path = ckpt
    got = C.from_pretrained(cfg, path)
    assert set(got) == set(sd)
    assert all(torch.equal(got[k], sd[k]) for k in sd)
    # a directory of shards
    raw = load_file(path)
    keys = sorted(raw)
    shard = tmp_path / 'shards'
    shard.mkdir()
    save_file({k: raw[k] for k in keys[::2]}, str(shard / 'a.safetensors'))
    save_file({k: raw[k] for k in keys[1::2]}, str(shard / 'b.safetensors'))
    got = C.from_pretrained(cfg, str(shard))
    assert all(torch.equal(got[k], sd[k]) for k in sd)
    # .pt, both {'model': sd} and a bare state dict
    for obj in ({'model': raw}, raw):
        pt = str(tmp_path / 'ck.pt')
        torch.save(obj, pt)
        got = C.from_pretrained(cfg, pt)
        assert all(torch.equal(got[k], sd[k]) for k in sd)


def test_mapping_errors_and_skips(ckpt):
    cfg, sd, path = ckpt
    raw = load_file(path)
    params = [(n, s) for n, s, _, _ in param_specs(cfg)]
    gone = 'paligemma_with_expert.gemma_expert.model.layers.0.mlp.up_proj.weight'
    partial = {k: v for k, v in raw.items() if k != gone}
    with pytest.raises(ValueError, match='not found'):
        C.map_state_dict(params, partial, C.PI0_NAME_MAPPING, strict=True)
    out, skipped = C.map_state_dict(params, partial, C.PI0_NAME_MAPPING,
                                    strict=False)
    assert skipped == ['llm_expert.layers.0.mlp.up_proj.weight']
    # a size mismatch is skipped, not copied
    bad = dict(raw)
    bad[gone] = torch.zeros(3, 3, dtype=torch.bfloat16)
    out, skipped = C.map_state_dict(params, bad, C.PI0_NAME_MAPPING,
                                    strict=False)
    assert 'llm_expert.layers.0.mlp.up_proj.weight' in skipped
    # two mapping pairs hitting existing checkpoint entries is an error
    # (llm_backbone.embed_tokens via 'llm_backbone' and via its own pair)
    dup = dict(raw)
    dup['paligemma_with_expert.paligemma.model.language_model.embed_tokens.weight'] = \
        raw['paligemma_with_expert.paligemma.lm_head.weight']
    with pytest.raises(ValueError, match='multiple'):
        C.map_state_dict(params, dup, C.PI0_NAME_MAPPING, strict=True)
    # without a mapping the names must match directly
    out, skipped = C.map_state_dict(params, sd, None, strict=True)
    assert all(torch.equal(out[k], sd[k]) for k in sd)


def test_from_pretrained_names_missing_parameters(ckpt, tmp_path):
    cfg, sd, path = ckpt
    raw = load_file(path)
    gone = 'paligemma_with_expert.gemma_expert.model.layers.0.mlp.up_proj.weight'
    p = str(tmp_path / 'partial.safetensors')
    save_file({k: v for k, v in raw.items() if k != gone}, p)
    with pytest.raises(ValueError, match='llm_expert.layers.0.mlp.up_proj'):
        C.from_pretrained(cfg, p)


def test_unsupported_format(tmp_path):
    p = tmp_path / 'x.bin'
    p.write_bytes(b'0')
    with pytest.raises(ValueError, match='Unsupported'):
        C.load_checkpoint(str(p))


def test_fp8_cache_source_hash(ckpt):
    cfg, sd, _ = ckpt
    h = C.source_hash(sd, cfg, 'bf16')
    assert h == C.source_hash(dict(sd), cfg, 'bf16')
    assert h != C.source_hash(sd, cfg, 'e4m3')
    sd2 = dict(sd)
    k = 'llm_expert.layers.0.mlp.down_proj.weight'
    sd2[k] = sd[k].clone()
    sd2[k][0, 0] += 1.0
    assert h != C.source_hash(sd2, cfg, 'bf16')
    assert h != C.source_hash(sd, cfg.scaled(rms_eps=1e-5), 'bf16')
