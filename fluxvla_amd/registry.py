"""Config-driven construction with the reference's type names.

The reference selects its model by ``inference_model=dict(type=...)`` through
``VLAS.register_module()`` / ``build_vla_from_cfg``
(fluxvla/engines/utils/registry.py:554-675, builder.py:317; e.g.
configs/pi0/pi0_paligemma_aloha_full_finetune.py:15-129,
configs/pi05/pi05_paligemma_libero_10_full_inference.py:118-181).  The same
config dicts build the HIP model here: the type name picks PI0 or PI0.5 and
the nested backbone dicts give the dimensions.
"""
from .config import PI0Config
from .pi0_inference import PI0Inference

VLAS = {}


def register_module(name=None):
    def deco(cls):
        VLAS[name or cls.__name__] = cls
        return cls
    return deco


@register_module()
class PI0FlowMatching(PI0Inference):
    """PI0 (state token, block-causal suffix, plain-RMSNorm expert)."""


@register_module()
class PI05FlowMatching(PI0Inference):
    """PI0.5 (adaRMS-conditioned expert, no state token)."""


@register_module()
class PI05FlowMatchingInference(PI0Inference):
    """The reference's fused PI0.5 inference type."""


PI05_TYPES = ('PI05FlowMatching', 'PI05FlowMatchingInference')


def config_from_reference(cfg: dict, num_views=None, max_prompt_len=None):
    """PI0Config from a reference model config dict (the dims it names)."""
    llm = cfg['llm_backbone']
    exp = cfg['llm_expert']
    vis = cfg['vision_backbone']['vision_config']
    pi05 = cfg['type'] in PI05_TYPES
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
        proj_width=cfg.get('proj_width', 1024),
        n_action_steps=cfg.get('n_action_steps', 50),
        max_action_dim=cfg.get('max_action_dim', 32),
        ori_action_dim=cfg.get('ori_action_dim'),
        num_steps=cfg.get('num_steps', 10), pi05=pi05)
    if not pi05 and cfg.get('state_proj'):
        kw['state_dim'] = cfg['state_proj']['in_dim']
    views = num_views if num_views is not None else cfg.get('num_views', 3)
    prompt = (max_prompt_len if max_prompt_len is not None else
              cfg.get('triton_max_prompt_len', 48))
    kw.update(n_views=views, max_prompt_len=prompt)
    if llm['num_hidden_layers'] != exp['num_hidden_layers']:
        raise ValueError('prefix LLM and action expert must have the same '
                         'number of layers (pi0_flowmatching.py:477-479)')
    return PI0Config(**kw)


def build_vla_from_cfg(cfg: dict, state_dict=None, device='cuda', max_batch=1,
                       num_views=None, max_prompt_len=None, use_graph=True,
                       **kwargs):
    """Build the registered inference model named by ``cfg['type']`` from a
    state dict with the reference's parameter names, or -- without one --
    from the config's ``pretrained_name_or_path`` through its
    ``name_mapping`` / ``strict_mapping`` (BaseVLA.from_pretrained,
    base_vla.py:190-288).  Extra keyword arguments go to the model
    (``weight_dtype``, ``fp8_cache``)."""
    name = cfg['type']
    if name not in VLAS:
        raise KeyError(f'{name} is not a registered VLA type '
                       f'({sorted(VLAS)})')
    pcfg = config_from_reference(cfg, num_views, max_prompt_len)
    if state_dict is None:
        from .checkpoint import from_pretrained
        path = cfg.get('pretrained_name_or_path')
        if not path:
            raise ValueError('no state_dict and no pretrained_name_or_path')
        state_dict = from_pretrained(pcfg, path, cfg.get('name_mapping'),
                                     strict=cfg.get('strict_mapping', False))
    return VLAS[name](pcfg, state_dict, device=device, max_batch=max_batch,
                      use_graph=use_graph, **kwargs)
