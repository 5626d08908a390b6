"""Seeded synthetic state dict and inputs for the PI0 / PI0.5 path.

Parameter names follow the reference's module tree (PI0FlowMatching with a
ConditionGemmaModel prefix LLM, an HF SiglipVisionModel tower under
``vision_backbone.vision`` and LinearProjector heads; fluxvla/models/vlas/
pi0_flowmatching.py:76-172, configs/pi0/pi0_paligemma_aloha_full_finetune.py
:15-129), so a checkpoint remapped with the reference's ``name_mapping`` has
the same keys.  There is no network here, so weights are random: linear
weights ~N(0, 0.02) like the HF initializer (condition_gemma.py:680-694),
biases ~N(0, 0.02), Gemma RMSNorm weights ~N(0, 0.1) (the (1 + w) scale then
varies by ~10 %), LayerNorm weights ~N(1, 0.05) and biases ~N(0, 0.02) --
non-trivial values so that the norm folds and bias epilogues are exercised.
"""
import hashlib

import torch

from .config import PI0Config

VIS = 'vision_backbone.vision.vision_model'


def param_specs(cfg: PI0Config):
    """[(name, shape, mean, std)] in a fixed order."""
    s = []

    def lin(name, n_out, n_in, bias):
        s.append((name + '.weight', (n_out, n_in), 0.0, 0.02))
        if bias:
            s.append((name + '.bias', (n_out, ), 0.0, 0.02))

    vh, p = cfg.vit_hidden, cfg.patch
    s.append((f'{VIS}.embeddings.patch_embedding.weight', (vh, 3, p, p), 0.0,
              0.02))
    s.append((f'{VIS}.embeddings.patch_embedding.bias', (vh, ), 0.0, 0.02))
    s.append((f'{VIS}.embeddings.position_embedding.weight',
              (cfg.num_patches, vh), 0.0, 0.02))
    for i in range(cfg.vit_layers):
        pre = f'{VIS}.encoder.layers.{i}'
        s.append((f'{pre}.layer_norm1.weight', (vh, ), 1.0, 0.05))
        s.append((f'{pre}.layer_norm1.bias', (vh, ), 0.0, 0.02))
        for nm in ('q_proj', 'k_proj', 'v_proj', 'out_proj'):
            lin(f'{pre}.self_attn.{nm}', vh, vh, True)
        s.append((f'{pre}.layer_norm2.weight', (vh, ), 1.0, 0.05))
        s.append((f'{pre}.layer_norm2.bias', (vh, ), 0.0, 0.02))
        lin(f'{pre}.mlp.fc1', cfg.vit_mlp, vh, True)
        lin(f'{pre}.mlp.fc2', vh, cfg.vit_mlp, True)
    s.append((f'{VIS}.post_layernorm.weight', (vh, ), 1.0, 0.05))
    s.append((f'{VIS}.post_layernorm.bias', (vh, ), 0.0, 0.02))
    lin('projector.projector', cfg.llm_hidden, vh, True)

    def gemma(prefix, hidden, mlp, n_layers, adarms):
        hq = cfg.heads * cfg.head_dim
        for i in range(n_layers):
            pre = f'{prefix}.layers.{i}'
            for norm in ('input_layernorm', 'post_attention_layernorm'):
                if adarms:
                    lin(f'{pre}.{norm}.dense', 3 * hidden, cfg.proj_width,
                        True)
                else:
                    s.append((f'{pre}.{norm}.weight', (hidden, ), 0.0, 0.1))
            lin(f'{pre}.self_attn.q_proj', hq, hidden, False)
            lin(f'{pre}.self_attn.k_proj', cfg.head_dim, hidden, False)
            lin(f'{pre}.self_attn.v_proj', cfg.head_dim, hidden, False)
            lin(f'{pre}.self_attn.o_proj', hidden, hq, False)
            lin(f'{pre}.mlp.gate_proj', mlp, hidden, False)
            lin(f'{pre}.mlp.up_proj', mlp, hidden, False)
            lin(f'{pre}.mlp.down_proj', hidden, mlp, False)
        if adarms:
            lin(f'{prefix}.norm.dense', 3 * hidden, cfg.proj_width, True)
        else:
            s.append((f'{prefix}.norm.weight', (hidden, ), 0.0, 0.1))

    s.append(('llm_backbone.embed_tokens.weight', (cfg.vocab, cfg.llm_hidden),
              0.0, 0.02))
    gemma('llm_backbone', cfg.llm_hidden, cfg.llm_mlp, cfg.llm_layers, False)
    gemma('llm_expert', cfg.exp_hidden, cfg.exp_mlp, cfg.exp_layers, cfg.pi05)

    w, ad = cfg.proj_width, cfg.max_action_dim
    lin('action_in_proj.projector', w, ad, True)
    lin('action_out_proj.projector', ad, cfg.exp_hidden, True)
    if cfg.pi05:
        lin('time_mlp_in.projector', w, w, True)
        lin('time_mlp_out.projector', w, w, True)
    else:
        lin('state_proj.projector', w, cfg.state_dim, True)
        lin('action_time_mlp_in.projector', w, 2 * w, True)
        lin('action_time_mlp_out.projector', w, w, True)
    return s


def _seed(base, name):
    h = hashlib.sha256(f'{base}:{name}'.encode()).digest()
    return int.from_bytes(h[:8], 'little') & ((1 << 62) - 1)


def make_state_dict(cfg: PI0Config, seed=0, device='cpu'):
    """bf16 parameters, each drawn from its own seeded generator on
    ``device`` (identical values for the same (seed, device type))."""
    dev = torch.device(device)
    sd = {}
    for name, shape, mean, std in param_specs(cfg):
        g = torch.Generator(device=dev).manual_seed(_seed(seed, name))
        t = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
        sd[name] = (t * std + mean).to(torch.bfloat16)
    return sd


def make_inputs(cfg: PI0Config, batch=1, seed=0, device='cpu'):
    """Synthetic request batch with the shapes PI0 predict_action takes
    (fluxvla/models/vlas/pi0_flowmatching.py:702-715): images are uint8
    uniform noise normalized to [-1, 1] as x / 127.5 - 1, all masks valid."""
    g = torch.Generator().manual_seed(seed)
    H = cfg.image_size
    img_u8 = torch.randint(0, 256, (batch, 3 * cfg.n_views, H, H),
                           generator=g, dtype=torch.uint8)
    images = img_u8.float() / 127.5 - 1.0
    lang_tokens = torch.randint(0, cfg.vocab, (batch, cfg.max_prompt_len),
                                generator=g, dtype=torch.int64)
    lang_masks = torch.ones(batch, cfg.max_prompt_len, dtype=torch.bool)
    img_masks = torch.ones(batch, cfg.n_views, dtype=torch.bool)
    states = torch.rand(batch, cfg.state_dim, generator=g) * 2 - 1
    noise = torch.randn(batch, cfg.n_action_steps, cfg.max_action_dim,
                        generator=g)
    out = dict(images=images, lang_tokens=lang_tokens, lang_masks=lang_masks,
               img_masks=img_masks, states=states, noise=noise)
    return {k: v.to(device) for k, v in out.items()}
