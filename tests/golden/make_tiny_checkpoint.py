"""Write a tiny PI0 / PI0.5 checkpoint in the reference's on-disk naming
(paligemma_with_expert.*, the names the PI0 configs' name_mapping points
to): the seeded synthetic state dict of a small config, exported through
fluxvla_amd.checkpoint.export_checkpoint.  Used by tests/test_checkpoint.py
(written into a temporary directory) and runnable by hand:

    python tests/golden/make_tiny_checkpoint.py OUT.safetensors [--pi05]
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def tiny_config(pi05=False):
    from fluxvla_amd.config import tiny
    return tiny(pi05=pi05, vit_hidden=64, vit_heads=4, vit_layers=1,
                vit_mlp=96, llm_hidden=64, llm_mlp=96, heads=4, head_dim=16,
                llm_layers=1, exp_hidden=32, exp_mlp=48, exp_layers=1,
                image_size=28, patch=14, proj_width=32, max_prompt_len=4)


def write(path, pi05=False, seed=5):
    """Export the synthetic state dict of tiny_config(pi05); returns
    (config, state dict)."""
    from fluxvla_amd.checkpoint import export_checkpoint
    from fluxvla_amd.weights import make_state_dict
    cfg = tiny_config(pi05)
    sd = make_state_dict(cfg, seed=seed)
    export_checkpoint(sd, path)
    return cfg, sd


if __name__ == '__main__':
    write(sys.argv[1], pi05='--pi05' in sys.argv)
