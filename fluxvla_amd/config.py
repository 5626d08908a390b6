"""Model dimensions of the PI0 / PI0.5 inference path.

Defaults are the reference's PI0 config (configs/pi0/
pi0_paligemma_aloha_full_finetune.py:15-129): SigLIP-So400m/14 at 224 px,
Gemma-2B prefix (width 2048, 18 layers, 8 query heads / 1 KV head, head_dim
256, GeGLU 16384), Gemma-300M action expert (width 1024, GeGLU 4096),
50-step action chunk of 32 dims, 10 Euler steps.
"""
from dataclasses import dataclass, replace
from typing import Optional


@dataclass(frozen=True)
class PI0Config:
    # camera views and SigLIP tower
    n_views: int = 3
    image_size: int = 224
    patch: int = 14
    vit_hidden: int = 1152
    vit_layers: int = 27
    vit_heads: int = 16
    vit_mlp: int = 4304
    vit_eps: float = 1e-6
    # Gemma-2B prefix LLM
    llm_hidden: int = 2048
    llm_layers: int = 18
    llm_mlp: int = 16384
    vocab: int = 257152
    # shared attention geometry (MQA)
    heads: int = 8
    head_dim: int = 256
    rms_eps: float = 1e-6
    rope_theta: float = 10000.0
    # Gemma-300M action expert
    exp_hidden: int = 1024
    exp_layers: int = 18
    exp_mlp: int = 4096
    # action head
    proj_width: int = 1024
    n_action_steps: int = 50
    max_action_dim: int = 32
    state_dim: int = 32
    num_steps: int = 10
    # PI0.5: adaRMS-conditioned expert, no state token
    pi05: bool = False
    # prompt length reserved in the static buffers
    max_prompt_len: int = 48
    # the robot's real action dims (pi0_flowmatching.py:108,168): shorter
    # previous chunks given for real-time chunking are zero-padded to
    # max_action_dim when set (:747-751)
    ori_action_dim: Optional[int] = None

    @property
    def num_patches(self):
        return (self.image_size // self.patch) ** 2

    @property
    def patch_k(self):
        return 3 * self.patch * self.patch

    @property
    def patch_k_pad(self):
        return (self.patch_k + 7) // 8 * 8

    @property
    def prefix_len(self):
        return self.n_views * self.num_patches + self.max_prompt_len

    @property
    def suffix_len(self):
        return self.n_action_steps + (0 if self.pi05 else 1)

    @property
    def vit_head_dim(self):
        return self.vit_hidden // self.vit_heads

    def scaled(self, **kw):
        return replace(self, **kw)


PI0 = PI0Config()
PI05 = PI0Config(pi05=True)


def tiny(pi05=False, **kw):
    """Real widths, few layers, small vocab: what CPU-oracle tests afford."""
    base = PI0Config(vit_layers=2, llm_layers=2, exp_layers=2, vocab=1024,
                     pi05=pi05)
    return replace(base, **kw)
