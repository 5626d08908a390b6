"""The reference's weight-preparation hooks, with its class names, method
signatures and dict keys.

* ``ConditionGemmaInferenceModel.prepare_triton(role)``
  (fluxvla/models/backbones/llms/condition_gemma_inference.py:65-170)
* ``SigLIPViTBackboneInference.prepare_triton()``
  (fluxvla/models/backbones/visions/siglip_vit_inference.py:10-101)
* ``LinearProjectorInference.prepare_triton(prefix)``
  (fluxvla/models/projectors/linear_projector_inference.py:8-14)

The reference's classes are nn.Modules holding their own parameters; here
each is built from a state dict with the reference's parameter names
(``from_state_dict``), which is what a checkpoint load produces.  Every
returned weight matrix is an ``NKWeight``: stored [out, in] for the HIP
GEMMs, presenting the reference's [in, out] shape and per-layer indexing
(``w[i]``), so the returned dicts drop into code written against the
reference's ``_triton_weights`` (pi05_flowmatching_inference.py:22-312, and
this package's mirror of it).  The folds are the reference's: Gemma (1 + w)
RMSNorm scales multiplied into Q/K/V and gate/up in fp32 before one bf16
rounding, Q/K rows in pair-interleaved RoPE order.
"""
import torch

from .config import PI0Config
from .pi0_inference import VIS, prepare_gemma, prepare_projector, prepare_siglip
from .weight_layout import NKWeight, PatchWeight

BF16 = torch.bfloat16


def _stack(layers, name):
    return torch.stack([L[name] for L in layers]).contiguous()


class LinearProjectorInference:
    """LinearProjectorInference: ``prepare_triton(prefix)`` returns
    ``{prefix + '_w': W [in, out], prefix + '_b': b}``."""

    def __init__(self, weight, bias, device='cuda'):
        self.weight, self.bias, self.device = weight, bias, device

    @classmethod
    def from_state_dict(cls, sd, module, device='cuda'):
        """``module``: the projector's name in the state dict, e.g.
        'projector' or 'action_in_proj' (its parameters are
        ``{module}.projector.weight`` / ``.bias``)."""
        return cls(sd[f'{module}.projector.weight'],
                   sd[f'{module}.projector.bias'], device)

    def prepare_triton(self, prefix='') -> dict:
        p = prepare_projector({'x.projector.weight': self.weight,
                               'x.projector.bias': self.bias}, 'x', self.device)
        return {f'{prefix}_w': NKWeight(p['w'].to(BF16)),
                f'{prefix}_b': p['b'].to(BF16)}


class SigLIPViTBackboneInference:
    """SigLIPViTBackboneInference: ``prepare_triton()`` returns the
    reference's ``vision_*`` keys (patch embedding, position embedding,
    per-layer QKV / O / fc1 ('ffn_up') / fc2 ('ffn_down') weights and
    biases, the two LayerNorms per layer and the final norm)."""

    def __init__(self, sd, cfg: PI0Config, device='cuda'):
        self.sd, self.cfg, self.device = sd, cfg, device

    @classmethod
    def from_state_dict(cls, sd, cfg, device='cuda'):
        return cls(sd, cfg, device)

    def prepare_triton(self) -> dict:
        cfg = self.cfg
        V = prepare_siglip(self.sd, cfg, self.device)
        L = V['layers']
        p = cfg.patch
        return {
            'vision_patch_embedding_w': PatchWeight(V['patch_w'], (p, p, 3)),
            'vision_patch_embedding_b': V['patch_b'],
            'vision_position_embedding': V['pos_emb'],
            'vision_attn_qkv_w': NKWeight(_stack(L, 'qkv_w')),
            'vision_attn_qkv_b': _stack(L, 'qkv_b'),
            'vision_attn_o_w': NKWeight(_stack(L, 'o_w')),
            'vision_attn_o_b': _stack(L, 'o_b'),
            'vision_ffn_up_w': NKWeight(_stack(L, 'fc1_w')),
            'vision_ffn_up_b': _stack(L, 'fc1_b'),
            'vision_ffn_down_w': NKWeight(_stack(L, 'fc2_w')),
            'vision_ffn_down_b': _stack(L, 'fc2_b'),
            'vision_pre_attn_norm_w': _stack(L, 'ln1_w'),
            'vision_pre_attn_norm_b': _stack(L, 'ln1_b'),
            'vision_pre_ffn_norm_w': _stack(L, 'ln2_w'),
            'vision_pre_ffn_norm_b': _stack(L, 'ln2_b'),
            'vision_final_norm_w': V['post_ln_w'],
            'vision_final_norm_b': V['post_ln_b'],
        }


class ConditionGemmaInferenceModel:
    """ConditionGemmaInferenceModel: ``prepare_triton(role)`` with role
    'llm' (the Gemma-2B prefix, ``encoder_*`` keys, RMSNorm scales folded)
    or 'expert' (the action expert, ``decoder_*`` keys).  An adaRMS expert
    (PI0.5) returns its modulation weights as the reference does
    (``decoder_pre_attn_norm_mod_w`` [L, cond, 3 width], ...,
    ``decoder_final_norm_mod_w``); a plain-RMSNorm expert (PI0, which the
    reference's fast path does not cover) gets its scales folded like the
    prefix and its final norm's (1 + w) as ``decoder_final_norm_scale``."""

    _PREFIX = {'llm': 'llm_backbone', 'expert': 'llm_expert'}

    def __init__(self, sd, cfg: PI0Config, module, device='cuda'):
        if module not in self._PREFIX.values():
            raise ValueError(f'module must be one of '
                             f'{sorted(self._PREFIX.values())}, got {module!r}')
        self.sd, self.cfg, self.module, self.device = sd, cfg, module, device

    @classmethod
    def from_state_dict(cls, sd, cfg, module, device='cuda'):
        return cls(sd, cfg, module, device)

    def prepare_triton(self, role='llm') -> dict:
        if role not in self._PREFIX:
            raise ValueError(f"role must be 'llm' or 'expert', got {role!r}")
        if self._PREFIX[role] != self.module:
            raise ValueError(f'role {role!r} prepares {self._PREFIX[role]}, '
                             f'this model is {self.module}')
        W = prepare_gemma(self.sd, self.cfg, role, self.device)
        L = W['layers']
        k = 'encoder' if role == 'llm' else 'decoder'
        out = {
            f'{k}_attn_qkv_w': NKWeight(_stack(L, 'qkv_w')),
            f'{k}_attn_o_w': NKWeight(_stack(L, 'o_w')),
            f'{k}_ffn_gate_w': NKWeight(_stack(L, 'gate_w')),
            f'{k}_ffn_up_w': NKWeight(_stack(L, 'up_w')),
            f'{k}_ffn_down_w': NKWeight(_stack(L, 'down_w')),
        }
        if role == 'expert':
            if 'attn_mod_w' in L[0]:
                out['decoder_pre_attn_norm_mod_w'] = NKWeight(_stack(L, 'attn_mod_w'))
                out['decoder_pre_attn_norm_mod_b'] = _stack(L, 'attn_mod_b')
                out['decoder_pre_ffn_norm_mod_w'] = NKWeight(_stack(L, 'ffn_mod_w'))
                out['decoder_pre_ffn_norm_mod_b'] = _stack(L, 'ffn_mod_b')
                out['decoder_final_norm_mod_w'] = NKWeight(W['final_mod_w'])
                out['decoder_final_norm_mod_b'] = W['final_mod_b']
            else:
                out['decoder_final_norm_scale'] = W['final_scale']
        return out


def reference_layout(weights):
    """A prepared-weights dict with every ``NKWeight`` replaced by the plain
    tensor the reference's own hooks would hand over ([in, out]; the patch
    weight [kH, kW, C, out]) -- for callers and tests that feed the ops the
    reference's layout."""
    return {k: v.reference() if isinstance(v, NKWeight) else v
            for k, v in weights.items()}


__all__ = ['ConditionGemmaInferenceModel', 'LinearProjectorInference',
           'SigLIPViTBackboneInference', 'reference_layout', 'VIS']
