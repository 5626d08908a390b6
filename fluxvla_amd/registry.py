"""Registered model types, built the way the reference's runners build them.

The reference names its model in the config (``inference_model=dict(
type='PI05FlowMatchingInference', ...)``) and its runners do, in order:

    vla = build_vla_from_cfg(cfg.inference_model)   # cls(**cfg without type)
    vla.load_state_dict(state_dict, strict=True)
    vla.eval(); vla.to(device)                      # or .to(device=, dtype=)
    actions = vla.predict_action(**batch)

(fluxvla/engines/utils/builder.py:26-110, 317-335;
fluxvla/engines/runners/serving/serve.py:45-66, zmq_server.py:208-209;
libero_eval_runner.py:89-95, 128, 170-181).  ``PI05FlowMatchingInference``
takes ``num_views``, ``triton_max_prompt_len`` and ``num_steps`` and
prepares its kernels' weights on the first ``predict_action``
(fluxvla/models/vlas/pi05_flowmatching_inference.py:342-356, 524-530).

The types here accept the same constructor arguments and the same call
sequence.  Construction holds no device memory and no weights;
``load_state_dict`` / ``from_pretrained`` keep a host copy of the state dict
(bf16, the reference's parameter names); the first ``predict_action``
builds a ``PI0Inference`` on the model's device (weight preparation, static
buffers, one HIP graph per batch size) and later calls replay it.  Loading
new weights or moving the model drops the prepared model, so no captured
graph ever reads stale weights.

``register_into(registry)`` registers the three types into a reference
``Registry`` (``fluxvla.engines.utils.root.VLAS``) under the reference's
names with ``force=True`` (fluxvla/engines/utils/registry.py:615-625), after
which the reference's own ``build_vla_from_cfg`` returns these classes.
``build_vla_from_cfg`` below does the same over this module's ``VLAS``.
"""
import collections

import torch

from .config import PI0Config
from .weights import param_specs

IncompatibleKeys = collections.namedtuple('IncompatibleKeys',
                                          ['missing_keys', 'unexpected_keys'])

# constructor arguments of the reference's PI0 / PI0.5 types that only
# concern training or the eager attention backend
# (pi0_flowmatching.py:76-110); accepted and recorded, no effect here
TRAINING_ARGS = frozenset({
    'vlm_backbone', 'vla_head', 'enable_mixed_precision_training',
    'freeze_vision_backbone', 'freeze_llm_backbone', 'freeze_vlm_backbone',
    'freeze_llm_expert', 'freeze_projector', 'vision_backbone_fp32',
    'unfreeze_last_layer', 'ignore_index', 'attention_implementation',
    'params_to_change_dtype', 'rtc_training_config',
    'action_in_proj', 'action_out_proj', 'projector', 'time_mlp_in',
    'time_mlp_out', 'action_time_mlp_in', 'action_time_mlp_out'})


def _pi0_config(pi05, llm_backbone, llm_expert, vision_backbone, proj_width,
                n_action_steps, max_action_dim, ori_action_dim, num_steps,
                state_proj, num_views, max_prompt_len):
    """PI0Config from the reference's nested config dicts."""
    llm, exp = llm_backbone, llm_expert
    vis = vision_backbone['vision_config']
    if llm['num_hidden_layers'] != exp['num_hidden_layers']:
        raise ValueError('prefix LLM and action expert must have the same '
                         'number of layers (pi0_flowmatching.py:477-479)')
    kw = dict(
        llm_hidden=llm['hidden_size'], llm_mlp=llm['intermediate_size'],
        llm_layers=llm['num_hidden_layers'],
        heads=llm['num_attention_heads'], head_dim=llm['head_dim'],
        rms_eps=llm.get('rms_norm_eps', 1e-6),
        rope_theta=llm.get('rope_theta', 10000.0),
        vocab=llm.get('vocab_size', 257152),
        exp_hidden=exp['hidden_size'], exp_mlp=exp['intermediate_size'],
        exp_layers=exp['num_hidden_layers'],
        vit_hidden=vis['hidden_size'], vit_mlp=vis['intermediate_size'],
        vit_layers=vis['num_hidden_layers'],
        vit_heads=vis['num_attention_heads'], image_size=vis['image_size'],
        patch=vis['patch_size'], vit_eps=vis.get('layer_norm_eps', 1e-6),
        proj_width=proj_width, n_action_steps=n_action_steps,
        max_action_dim=max_action_dim, ori_action_dim=ori_action_dim,
        num_steps=num_steps, pi05=pi05, n_views=num_views,
        max_prompt_len=max_prompt_len)
    if not pi05 and state_proj:
        kw['state_dim'] = state_proj['in_dim']
    return PI0Config(**kw)


def _parse_to(args, kwargs):
    """(device, dtype) from nn.Module.to's call forms: to(device),
    to(dtype), to(device, dtype), to(tensor), keywords."""
    device = kwargs.pop('device', None)
    dtype = kwargs.pop('dtype', None)
    kwargs.pop('non_blocking', None)
    if kwargs:
        raise TypeError(f'to() got unexpected arguments {sorted(kwargs)}')
    for a in args:
        if isinstance(a, torch.dtype):
            dtype = a
        elif isinstance(a, torch.Tensor):
            device, dtype = a.device, a.dtype
        elif a is not None:
            device = a
    if isinstance(device, int):
        device = torch.device('cuda', device)
    return (None if device is None else torch.device(device)), dtype


class FlowMatchingInference:
    """A registered PI0 / PI0.5 type: the reference's constructor
    arguments, state-dict protocol and ``predict_action``."""

    pi05 = False
    # the reference's fused type reads num_views / triton_max_prompt_len
    # (defaults 2 / 48); the eager types take the view count and prompt
    # length from the first request
    fused = False

    def __init__(self, llm_backbone, llm_expert, vision_backbone,
                 proj_width=1024, n_action_steps=50, max_action_dim=32,
                 ori_action_dim=None, num_steps=10, state_proj=None,
                 num_views=None, triton_max_prompt_len=None,
                 pretrained_name_or_path=None, name_mapping=None,
                 strict_mapping=False, norm_stats=None, weight_dtype='bf16',
                 fp8_cache=None, use_graph=True, **kwargs):
        unknown = set(kwargs) - TRAINING_ARGS
        if unknown:
            raise TypeError(f'{type(self).__name__} got unexpected config '
                            f'keys {sorted(unknown)}')
        self._dims = dict(llm_backbone=llm_backbone, llm_expert=llm_expert,
                          vision_backbone=vision_backbone,
                          proj_width=proj_width, n_action_steps=n_action_steps,
                          max_action_dim=max_action_dim,
                          ori_action_dim=ori_action_dim, num_steps=num_steps,
                          state_proj=state_proj)
        if self.fused:
            num_views = 2 if num_views is None else num_views
            triton_max_prompt_len = (48 if triton_max_prompt_len is None
                                     else triton_max_prompt_len)
        self.num_views = num_views
        self.triton_max_prompt_len = triton_max_prompt_len
        self.num_steps = num_steps
        self.n_action_steps = n_action_steps
        self.max_action_dim = max_action_dim
        self.ori_action_dim = ori_action_dim
        self.pretrained_name_or_path = pretrained_name_or_path
        self.name_mapping = name_mapping
        self.strict_mapping = strict_mapping
        self.norm_stats = norm_stats
        self.training_args = dict(kwargs)
        self.weight_dtype = weight_dtype
        self.fp8_cache = fp8_cache
        self.use_graph = use_graph
        self.device = torch.device('cpu')
        self.training = False
        self._sd = None
        self._model = None
        # a config with the request-dependent sizes at their defaults: the
        # parameter names and shapes do not depend on them
        self.config = self._config(num_views or 3,
                                   triton_max_prompt_len or 48)

    def _config(self, views, prompt_len):
        return _pi0_config(self.pi05, num_views=views,
                           max_prompt_len=prompt_len, **self._dims)

    # -- nn.Module protocol ---------------------------------------------------
    def parameter_shapes(self):
        """{name: shape} of the parameters the model needs (the reference's
        module tree; weights.param_specs)."""
        return {n: tuple(s) for n, s, _, _ in param_specs(self.config)}

    def state_dict(self):
        """The loaded parameters (host, bf16), or an empty dict."""
        return dict(self._sd or {})

    def load_state_dict(self, state_dict, strict=True, assign=False):
        """nn.Module.load_state_dict: names and shapes are checked against
        the model's parameters; with ``strict`` a missing or unexpected key
        raises.  A shape mismatch always raises.  The tensors are kept on
        the host in bf16; the next predict_action prepares them."""
        want = self.parameter_shapes()
        missing = [k for k in want if k not in state_dict]
        unexpected = [k for k in state_dict if k not in want]
        errors = []
        if strict:
            if unexpected:
                errors.append('Unexpected key(s) in state_dict: ' +
                              ', '.join(f'"{k}"' for k in unexpected[:8]) +
                              (' ...' if len(unexpected) > 8 else ''))
            if missing:
                errors.append('Missing key(s) in state_dict: ' +
                              ', '.join(f'"{k}"' for k in missing[:8]) +
                              (' ...' if len(missing) > 8 else ''))
        for k, shape in want.items():
            t = state_dict.get(k)
            if t is not None and tuple(t.shape) != shape:
                errors.append(f'size mismatch for {k}: copying a param with '
                              f'shape {tuple(t.shape)} from checkpoint, the '
                              f'shape in current model is {shape}.')
        if errors:
            raise RuntimeError(f'Error(s) in loading state_dict for '
                               f'{type(self).__name__}:\n\t' +
                               '\n\t'.join(errors))
        sd = dict(self._sd or {})
        for k in want:
            if k in state_dict:
                sd[k] = state_dict[k].detach().to('cpu', torch.bfloat16)
        self._sd = sd
        self._model = None
        return IncompatibleKeys(missing, unexpected)

    def from_pretrained(self):
        """BaseVLA.from_pretrained (base_vla.py:190-288):
        ``pretrained_name_or_path`` through ``name_mapping``."""
        if self.pretrained_name_or_path is None:
            return
        from .checkpoint import from_pretrained
        sd = from_pretrained(self.config, self.pretrained_name_or_path,
                             self.name_mapping, strict=self.strict_mapping)
        self.load_state_dict(sd, strict=True)

    def eval(self):
        return self.train(False)

    def train(self, mode=True):
        if mode:
            raise RuntimeError(f'{type(self).__name__} is an inference model '
                               '(no training path)')
        self.training = False
        return self

    def requires_grad_(self, requires_grad=True):
        return self

    def to(self, *args, **kwargs):
        """Moves the model to a device (a GPU for predict_action).  The
        arithmetic is the reference's mixed-precision one whatever dtype is
        asked for: bf16 weights and activations, fp32 accumulation, fp32
        Euler state; float16 has no path and is refused."""
        device, dtype = _parse_to(args, kwargs)
        if dtype is not None and dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f'{type(self).__name__} computes in bf16 '
                             f'(fp32 accumulation); dtype {dtype} has no path')
        if device is not None:
            if device.type == 'cuda' and device.index is None:
                device = torch.device('cuda', torch.cuda.current_device())
            if device != self.device:
                self._model = None
            self.device = device
        return self

    def cuda(self, device=None):
        return self.to(torch.device('cuda', device) if isinstance(device, int)
                       else (device or 'cuda'))

    def cpu(self):
        return self.to('cpu')

    # -- inference ------------------------------------------------------------
    def _ensure_model(self, n_views, prompt_len, batch):
        from .pi0_inference import PI0Inference
        if self.device.type != 'cuda':
            raise RuntimeError(f'{type(self).__name__} runs on the GPU; '
                               f'move it there with .to("cuda") (it is on '
                               f'{self.device})')
        m = self._model
        if m is not None and (m.cfg.n_views != n_views or
                              m.cfg.max_prompt_len < prompt_len):
            m = None
        if m is None:
            cfg = self._config(n_views, prompt_len)
            m = PI0Inference(cfg, self._sd, device=self.device,
                             max_batch=batch, use_graph=self.use_graph,
                             weight_dtype=self.weight_dtype,
                             fp8_cache=self.fp8_cache)
            self._model = m
        m.max_batch = max(m.max_batch, batch)
        return m

    @property
    def inference_model(self):
        """The prepared PI0Inference (None before the first predict_action
        or after new weights / a device move)."""
        return self._model

    def predict_action(self, images, lang_tokens, states, img_masks=None,
                       lang_masks=None, past_key_values=None, noise=None,
                       *args, **kwargs):
        """pi0_flowmatching.py:702-715 (real-time chunking keywords
        included): [B, n_action_steps, max_action_dim] float32 on the
        model's device.  The reference's fused PI0.5 type serves batch item
        0 only and returns [1, ...]; here every item of the batch is
        denoised (the same result at B = 1)."""
        if self._sd is None:
            raise RuntimeError(f'{type(self).__name__}: no weights; call '
                               'load_state_dict() or from_pretrained() '
                               'first')
        n_views = images.shape[1] // 3
        if self.fused:
            if n_views != self.num_views:
                raise ValueError(f'{n_views} views given, the model was '
                                 f'configured with num_views='
                                 f'{self.num_views}')
            prompt_len = self.triton_max_prompt_len
        else:
            # the prompt buffer covers the last valid token of the batch
            # (ProcessPrompts pads far past it), rounded up to 16 and at
            # least the fused type's default of 48
            used = lang_tokens.shape[1]
            if lang_masks is not None and lang_masks.shape[1] > 0:
                valid = lang_masks.bool().any(0).nonzero()
                used = int(valid.max()) + 1 if valid.numel() else 1
            prompt_len = max((used + 15) // 16 * 16,
                             self.triton_max_prompt_len or 48)
        m = self._ensure_model(n_views, prompt_len, images.shape[0])
        return m.predict_action(images, lang_tokens, states, img_masks,
                                lang_masks, past_key_values, noise, *args,
                                **kwargs)

    # -- the reference's prepare hooks over the loaded weights -----------------
    def _hook_model(self):
        if self._sd is None:
            raise RuntimeError('no weights loaded')
        return self.config, self._sd

    @property
    def vision_backbone(self):
        from .hooks import SigLIPViTBackboneInference
        cfg, sd = self._hook_model()
        return SigLIPViTBackboneInference(sd, cfg, self.device)

    @property
    def llm_backbone(self):
        from .hooks import ConditionGemmaInferenceModel
        cfg, sd = self._hook_model()
        return ConditionGemmaInferenceModel(sd, cfg, 'llm_backbone',
                                            self.device)

    @property
    def llm_expert(self):
        from .hooks import ConditionGemmaInferenceModel
        cfg, sd = self._hook_model()
        return ConditionGemmaInferenceModel(sd, cfg, 'llm_expert', self.device)

    @property
    def projector(self):
        from .hooks import LinearProjectorInference
        _, sd = self._hook_model()
        return LinearProjectorInference.from_state_dict(sd, 'projector',
                                                        self.device)


VLAS = {}


def register_module(name=None):
    def deco(cls):
        VLAS[name or cls.__name__] = cls
        return cls
    return deco


@register_module()
class PI0FlowMatching(FlowMatchingInference):
    """PI0 (state token, block-causal suffix, plain-RMSNorm expert)."""


@register_module()
class PI05FlowMatching(FlowMatchingInference):
    """PI0.5 (adaRMS-conditioned expert, no state token)."""
    pi05 = True


@register_module()
class PI05FlowMatchingInference(FlowMatchingInference):
    """The reference's fused PI0.5 inference type."""
    pi05 = True
    fused = True


PI05_TYPES = tuple(n for n, c in VLAS.items() if c.pi05)


def register_into(registry, force=True):
    """Register the types into a reference ``Registry`` (e.g.
    ``fluxvla.engines.utils.root.VLAS``) under the reference's names, with
    its ``register_module(name=..., force=..., module=...)`` call
    (fluxvla/engines/utils/registry.py:615-625)."""
    for name, cls in VLAS.items():
        registry.register_module(name=name, force=force, module=cls)
    return registry


def config_from_reference(cfg: dict, num_views=None, max_prompt_len=None):
    """PI0Config from a reference model config dict (``type`` plus the
    constructor arguments)."""
    kw = {k: v for k, v in cfg.items() if k != 'type'}
    model = VLAS[cfg['type']](**kw) if cfg['type'] in VLAS else None
    if model is None:
        raise KeyError(f'{cfg["type"]} is not a registered VLA type '
                       f'({sorted(VLAS)})')
    views = num_views or model.num_views or 3
    prompt = max_prompt_len or model.triton_max_prompt_len or 48
    return model._config(views, prompt)


def build_vla_from_cfg(cfg: dict, default_args=None):
    """builder.build_vla_from_cfg (builder.py:26-110, 317-335) over this
    module's registry: ``cls(**cfg without 'type')``, default_args filling
    what cfg leaves out.  No weights are loaded (the caller's
    load_state_dict / from_pretrained does that)."""
    args = dict(default_args or {})
    args.update(cfg)
    name = args.pop('type', None)
    if name is None:
        raise KeyError('`cfg` or `default_args` must contain the key "type"')
    cls = VLAS.get(name) if isinstance(name, str) else name
    if cls is None:
        raise KeyError(f'{name} is not a registered VLA type '
                       f'({sorted(VLAS)})')
    return cls(**args)
