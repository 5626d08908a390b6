"""Weight ingestion: checkpoints into the inference model, and the offline
fp8 quantization cache.

``load_checkpoint`` / ``from_pretrained`` follow ``BaseVLA.from_pretrained``
(fluxvla/models/vlas/base_vla.py:190-288): a ``.safetensors`` file, a
directory of them, or a ``.pt`` / ``.pth`` file (``{'model': sd}`` or a bare
state dict); then every model parameter is looked up through
``name_mapping`` exactly as the reference does -- for each (key, value)
pair whose key occurs in the parameter name, ``name.replace(key, value)``
is tried in the checkpoint; a parameter matched by two pairs is an error, a
size mismatch is skipped, and with ``strict`` an unmatched parameter is an
error.  ``PI0_NAME_MAPPING`` is the mapping of the reference's PI0 / PI0.5
configs (configs/pi0/pi0_paligemma_aloha_full_finetune.py:106-119).  The
model's parameter names and shapes come from ``weights.param_specs`` (the
reference's module tree).  Checkpoints are read with loaders that execute
nothing from the file (safetensors; ``torch.load(weights_only=True)``).

``build_fp8_cache`` / ``load_fp8_cache``: the fp8 variant quantizes every
Gemma linear after the preparation folds (per-output-channel scale, e4m3
bytes); the cache keeps those bytes and scales in a safetensors file next
to a hash of the source weights and the model config, so a later process
loads them instead of quantizing, and a changed source is never served a
stale cache.
"""
import hashlib
import json
import os

import torch

from .config import PI0Config
from .weights import param_specs

PI0_NAME_MAPPING = {
    'llm_backbone': 'paligemma_with_expert.paligemma.model.language_model',
    'vision_backbone.vision':
    'paligemma_with_expert.paligemma.model.vision_tower',
    'projector.projector':
    'paligemma_with_expert.paligemma.model.multi_modal_projector.linear',
    'llm_expert': 'paligemma_with_expert.gemma_expert.model',
    'action_time_mlp_in.projector': 'action_time_mlp_in',
    'action_time_mlp_out.projector': 'action_time_mlp_out',
    'state_proj.projector': 'state_proj',
    'action_in_proj.projector': 'action_in_proj',
    'action_out_proj.projector': 'action_out_proj',
    'llm_backbone.embed_tokens': 'paligemma_with_expert.paligemma.lm_head',
}


def load_checkpoint(path):
    """The raw checkpoint dict: safetensors file or directory (every
    ``*.safetensors`` in it, in sorted order), or a ``.pt`` / ``.pth`` file
    (``{'model': sd}`` or ``sd``; weights_only, nothing executed)."""
    from safetensors.torch import load_file
    if path.endswith('.safetensors'):
        return load_file(path, device='cpu')
    if os.path.isdir(path):
        out = {}
        for f in sorted(os.listdir(path)):
            if f.endswith('.safetensors'):
                out.update(load_file(os.path.join(path, f), device='cpu'))
        if not out:
            raise ValueError(f'no .safetensors files in {path}')
        return out
    if path.endswith('.pt') or path.endswith('.pth'):
        ck = torch.load(path, map_location='cpu', weights_only=True)
        if isinstance(ck, dict) and 'model' in ck:
            ck = ck['model']
        return ck
    raise ValueError(f'Unsupported checkpoint format: {path}')


def map_state_dict(params, ckpt, name_mapping=None, strict=True,
                   dtype=torch.bfloat16):
    """Model state dict ``{name: tensor}`` for ``params`` ([(name, shape)])
    from ``ckpt`` through ``name_mapping`` (base_vla.py:221-288).  Without a
    mapping the names must match directly.  Returns (state dict, skipped
    names)."""
    sd, skipped = {}, []
    for name, shape in params:
        shape = tuple(shape)
        if not name_mapping:
            t = ckpt.get(name)
            if t is None or tuple(t.shape) != shape:
                if strict:
                    raise ValueError(f"Parameter '{name}' not found in "
                                     'pretrained weights.')
                skipped.append(name)
                continue
            sd[name] = t.to(dtype)
            continue
        matched = False
        for key, val in name_mapping.items():
            if key not in name:
                continue
            mapped = name.replace(key, val)
            if mapped not in ckpt:
                continue
            if matched:
                raise ValueError(f"Parameter '{name}' matched multiple times "
                                 'in name_mapping.')
            t = ckpt[mapped]
            if tuple(t.shape) != shape:
                continue  # size mismatch: skipped, as the reference does
            sd[name] = t.to(dtype)
            matched = True
        if not matched:
            if strict:
                raise ValueError(f"Parameter '{name}' not found in pretrained "
                                 'weights with mapping.')
            skipped.append(name)
    return sd, skipped


def from_pretrained(cfg: PI0Config, path, name_mapping=PI0_NAME_MAPPING,
                    strict=False, dtype=torch.bfloat16):
    """State dict of the PI0 / PI0.5 model ``cfg`` from a checkpoint.
    ``strict`` defaults to the reference's ``strict_mapping=False``
    (base_vla.py:55): unmatched parameters are collected rather than raised
    one by one -- but the inference model has no initialized fallback for
    them, so any left over is an error naming them all."""
    params = [(n, s) for n, s, _, _ in param_specs(cfg)]
    sd, skipped = map_state_dict(params, load_checkpoint(path), name_mapping,
                                 strict, dtype)
    if skipped:
        raise ValueError(f'{len(skipped)} parameters not found in {path} '
                         f'(after name_mapping): {skipped[:8]}'
                         + (' ...' if len(skipped) > 8 else ''))
    return sd


def export_checkpoint(sd, path, name_mapping=PI0_NAME_MAPPING):
    """Write a state dict under the checkpoint names ``name_mapping`` maps
    its parameters to, as a safetensors file: the inverse of
    from_pretrained.  A parameter several keys match takes the longest
    (most specific) one -- e.g. the prefix LLM's embedding table goes to
    ``lm_head`` as in the reference's checkpoints, not under the generic
    ``llm_backbone`` pair."""
    from safetensors.torch import save_file
    out = {}
    for name, t in sd.items():
        keys = [k for k in (name_mapping or {}) if k in name]
        mapped = name
        if keys:
            key = max(keys, key=len)
            mapped = name.replace(key, name_mapping[key])
        out[mapped] = t.detach().cpu().contiguous()
    save_file(out, path)


# ---------------------------------------------------------------------------
# fp8 quantization cache
# ---------------------------------------------------------------------------
FP8_CACHE_VERSION = 1


def source_hash(sd, cfg: PI0Config, act):
    """sha256 over the model config, the activation mode and every tensor
    of ``sd`` the fp8 preparation reads (names, shapes, dtypes, bytes)."""
    h = hashlib.sha256()
    h.update(json.dumps({'v': FP8_CACHE_VERSION, 'act': act,
                         'cfg': repr(cfg)}, sort_keys=True).encode())
    for name in sorted(sd):
        if not (name.startswith('llm_backbone.layers.') or
                name.startswith('llm_expert.layers.')):
            continue
        t = sd[name].detach().cpu().contiguous()
        h.update(name.encode())
        h.update(repr((tuple(t.shape), str(t.dtype))).encode())
        h.update(t.view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def _fp8_tensors(model):
    out = {}
    for role, W in (('llm', model.llm), ('expert', model.exp)):
        for i, L in enumerate(W['layers']):
            for nm in ('qkv_w', 'o_w', 'gate_w', 'up_w', 'down_w'):
                w = L[nm]
                out[f'{role}.{i}.{nm}.data'] = w.data.detach().cpu().contiguous()
                out[f'{role}.{i}.{nm}.scale'] = w.scale.detach().cpu().contiguous()
    return out


def build_fp8_cache(model, sd, path):
    """Write the fp8 model's quantized Gemma linears (row-major e4m3 bytes
    and fp32 scales, after the preparation folds) to ``path``
    (safetensors), with the source hash in its metadata."""
    from safetensors.torch import save_file
    if not model.fp8:
        raise ValueError('build_fp8_cache needs an fp8 model')
    act = 'e4m3' if model.weight_dtype == 'fp8_w8a8' else 'bf16'
    meta = {'source_sha256': source_hash(sd, model.cfg, act), 'act': act,
            'version': str(FP8_CACHE_VERSION)}
    save_file(_fp8_tensors(model), path, metadata=meta)
    return meta['source_sha256']


def load_fp8_cache(path, sd, cfg: PI0Config, act, device):
    """{role: [layer dicts of Fp8Weight]} from a cache written for exactly
    this source (``sd``, ``cfg``, ``act``); None if the file is absent or was
    written for other weights."""
    from safetensors import safe_open

    from .kernels import Fp8Weight
    if not os.path.exists(path):
        return None
    with safe_open(path, framework='pt', device='cpu') as f:
        meta = f.metadata() or {}
        if (meta.get('version') != str(FP8_CACHE_VERSION) or meta.get('act') != act
                or meta.get('source_sha256') != source_hash(sd, cfg, act)):
            return None
        out = {}
        for role, n in (('llm', cfg.llm_layers), ('expert', cfg.exp_layers)):
            layers = []
            for i in range(n):
                L = {}
                for nm in ('qkv_w', 'o_w', 'gate_w', 'up_w', 'down_w'):
                    data = f.get_tensor(f'{role}.{i}.{nm}.data').to(device)
                    scale = f.get_tensor(f'{role}.{i}.{nm}.scale').to(device)
                    L[nm] = Fp8Weight(data.contiguous(), scale.contiguous(),
                                      data.shape[0], data.shape[1], act=act)
                layers.append(L)
            out[role] = layers
    return out
