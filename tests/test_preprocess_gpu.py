"""fvx_resize_normalize (fluxvla_amd/preprocess.py) against the CPU
restatement of the reference's host transforms (oracle/preprocess_oracle.py).

Bars: the Pillow path is bit-exact in uint8 (read back through an identity
normalization); the bilinear path is within one uint8 level of the rounded
torch interpolate (exact where no rounding tie is near); normalized outputs
within 1e-5 of numpy's float32 arithmetic on the same resized pixels; pad
placement exact.
"""
import numpy as np
import pytest
import torch

from oracle import preprocess_oracle as PO
from tests.conftest import announce

pytestmark = pytest.mark.gpu

MEANS = [[123.515625, 116.04492188, 103.59375]] * 3
STDS = [[58.27148438, 57.02636719, 57.27539062]] * 3


def frames(seed, n, h, w):
    g = torch.Generator().manual_seed(seed)
    # smooth content plus noise, so interpolation weights matter
    yy = torch.linspace(0, 6.28, h)[:, None, None]
    xx = torch.linspace(0, 6.28, w)[None, :, None]
    base = 127 + 100 * torch.sin(yy * torch.tensor([1.0, 2.0, 3.0]) + xx)
    noise = torch.randint(-20, 21, (n, h, w, 3), generator=g)
    return (base[None] + noise).clamp(0, 255).to(torch.uint8)


@pytest.fixture(scope='module')
def P():
    from fluxvla_amd import preprocess
    from fluxvla_amd import kernels
    kernels._lib.load()
    return preprocess


@pytest.mark.parametrize('h,w', [(480, 640), (224, 224), (120, 160), (300, 250)])
def test_pil_bilinear_bit_exact(P, cuda, h, w):
    """TransformImage resize-naive: Pillow BILINEAR, every pixel equal."""
    announce(f'resize pil {h}x{w} -> 224x224')
    src = frames(1, 2, h, w)
    pre = P.ImagePreprocessor(224, 224, resize='pil')
    got = pre([src.to(cuda)]).cpu()
    for i in range(2):
        ref = PO.resize_pil_u8(src[i].numpy(), 224, 224)
        assert np.array_equal(got[i].permute(1, 2, 0).numpy(),
                              ref.astype(np.float32)), i


@pytest.mark.parametrize('h,w', [(480, 640), (224, 224), (120, 160), (333, 517)])
def test_linear_resize_normalize(P, cuda, h, w):
    """ResizeImages + NormalizeImages for three views of different sizes'
    worth: uint8 within one level, then numpy's normalization."""
    announce(f'resize linear {h}x{w} -> 224x224 + normalize')
    views = [frames(10 + v, 2, h, w) for v in range(3)]
    pre = P.ImagePreprocessor.from_transforms([
        dict(type='ResizeImages', height=224, width=224),
        dict(type='NormalizeImages', means=MEANS, stds=STDS)])
    got = pre([v.to(cuda) for v in views]).cpu().numpy()
    raw = P.ImagePreprocessor(224, 224, resize='linear')(
        [v.to(cuda) for v in views]).cpu().numpy()
    for b in range(2):
        r8 = np.stack([PO.resize_linear_u8(views[v][b].numpy(), 224, 224)
                       .transpose(2, 0, 1) for v in range(3)])
        g8 = raw[b].reshape(3, 3, 224, 224)
        diff = np.abs(g8 - r8.astype(np.float32))
        assert diff.max() <= 1.0
        assert (diff > 0).mean() < 1e-3
        # normalization of the kernel's own resized pixels, numpy float32
        ref = PO.normalize_images(g8, MEANS, STDS)
        assert np.abs(got[b].reshape(3, 3, 224, 224) - ref).max() <= 1e-5


def test_linear_fp32_matches_interpolate(P, cuda):
    """fp32 sources: torch bilinear interpolate, no rounding."""
    announce('resize linear fp32 planar 97x131 -> 60x50')
    g = torch.Generator().manual_seed(3)
    src = torch.rand(2, 3, 97, 131, generator=g) * 2 - 1
    out = torch.empty(2, 3, 60, 50, device=cuda)
    from fluxvla_amd import kernels as K
    K.resize_normalize(src.to(cuda), out, hwc=False)
    ref = torch.nn.functional.interpolate(src, size=(60, 50), mode='bilinear',
                                          align_corners=False)
    assert (out.cpu() - ref).abs().max().item() <= 1e-5


@pytest.mark.parametrize('direction', ['center', 'top-left', 'bottom-right',
                                       'top-right'])
def test_resize_with_pad_directions(P, cuda, direction):
    """ResizeImagesWithPad: aspect kept, pad placement per direction."""
    announce(f'resize with pad 300x480 -> 224x224 {direction}')
    src = frames(5, 1, 300, 480)
    pre = P.ImagePreprocessor(224, 224, resize='pad', pad_value=0,
                              pad_direction=direction)
    got = pre([src.to(cuda)]).cpu()[0].numpy()
    ref = PO.resize_chw_with_pad(src[0].permute(2, 0, 1).numpy(), 224, 224, 0,
                                 direction).astype(np.float32)
    diff = np.abs(got - ref)
    assert diff.max() <= 1.0 and (diff > 0).mean() < 1e-3
    # 300 x 480 -> 140 x 224: 84 pad rows, split per direction, exactly 0
    top = {'center': 42, 'top-left': 84, 'top-right': 84,
           'bottom-right': 0}[direction]
    pad_rows = np.r_[0:top, top + 140:224]
    assert np.all(got[:, pad_rows] == 0.0)
    assert got[:, top:top + 140].max() > 0


def test_model_utils_resize_with_pad(P, cuda):
    """model_utils.resize_with_pad: float images, pad -1 on the left/top."""
    announce('model_utils resize_with_pad 2x3x180x320 -> 224x224')
    g = torch.Generator().manual_seed(6)
    img = torch.rand(2, 3, 180, 320, generator=g) * 2 - 1
    got = P.resize_with_pad(img.to(cuda), 224, 224).cpu()
    ref = PO.resize_with_pad(img, 224, 224)
    assert got.shape == ref.shape
    assert (got - ref).abs().max().item() <= 1e-5


def test_swap_rb_and_planar_source(P, cuda):
    """BGR frames with swap_rb equal RGB frames; planar uint8 sources equal
    interleaved ones."""
    announce('resize swap_rb + planar')
    src = frames(7, 1, 240, 320)
    pre = P.ImagePreprocessor(224, 224, resize='linear')
    rgb = pre([src.to(cuda)]).cpu()
    bgr = P.ImagePreprocessor(224, 224, resize='linear', swap_rb=True)(
        [src.flip(-1).contiguous().to(cuda)]).cpu()
    assert torch.equal(rgb, bgr)
    planar = pre([src.permute(0, 3, 1, 2).contiguous().to(cuda)], hwc=False).cpu()
    assert torch.equal(rgb, planar)


def test_preprocessed_frames_feed_the_model(P, cuda):
    """Camera frames -> device preprocessing -> chunk graph, against the
    oracle chunk on the host transforms' images (max abs error 2e-2)."""
    announce('preprocess -> predict_action vs oracle')
    from fluxvla_amd.config import tiny
    from fluxvla_amd.pi0_inference import PI0Inference
    from fluxvla_amd.weights import make_inputs, make_state_dict
    from oracle import pi0_oracle as O
    cfg = tiny(vit_layers=1, llm_layers=1, exp_layers=1)
    sd = make_state_dict(cfg, seed=2)
    m = PI0Inference(cfg, sd, device='cuda')
    inp = make_inputs(cfg, batch=1, seed=3)
    views = [frames(20 + v, 1, 480, 640) for v in range(3)]
    pre = P.ImagePreprocessor.from_transforms([
        dict(type='ResizeImages', height=224, width=224),
        dict(type='NormalizeImages', means=MEANS, stds=STDS)])
    got = m.predict_action(pre([v.to(cuda) for v in views]),
                           inp['lang_tokens'].to(cuda), inp['states'].to(cuda),
                           noise=inp['noise'].to(cuda)).cpu()
    r8 = np.stack([PO.resize_linear_u8(views[v][0].numpy(), 224, 224)
                   .transpose(2, 0, 1) for v in range(3)])
    imgs = torch.from_numpy(PO.normalize_images(r8, MEANS, STDS)).reshape(
        1, 9, 224, 224)
    ref = O.predict_action(sd, cfg, imgs, inp['lang_tokens'], inp['states'],
                           noise=inp['noise'])
    err = (got - ref).abs().max().item()
    print(f'chunk max abs err {err:.3e}')
    assert err <= 2e-2


def test_prompt_padded_past_buffer_is_trimmed(P, cuda):
    """ProcessPrompts pads to 180 tokens by default: padding past the
    model's prompt buffer is dropped (same chunk); real tokens past it are
    refused."""
    announce('prompt padded to 180 tokens')
    from fluxvla_amd.config import tiny
    from fluxvla_amd.pi0_inference import PI0Inference
    from fluxvla_amd.weights import make_inputs, make_state_dict
    cfg = tiny(vit_layers=1, llm_layers=1, exp_layers=1)
    m = PI0Inference(cfg, make_state_dict(cfg, seed=4), device='cuda')
    inp = make_inputs(cfg, batch=1, seed=5)
    toks, mask = inp['lang_tokens'].clone(), inp['lang_masks'].clone()
    mask[:, 30:] = False
    long_t = torch.zeros(1, 180, dtype=torch.int64)
    long_m = torch.zeros(1, 180, dtype=torch.bool)
    long_t[:, :48], long_m[:, :48] = toks, mask
    args = (inp['images'].to(cuda), )
    a = m.predict_action(*args, toks.to(cuda), inp['states'].to(cuda),
                         lang_masks=mask.to(cuda), noise=inp['noise'].to(cuda))
    b = m.predict_action(*args, long_t.to(cuda), inp['states'].to(cuda),
                         lang_masks=long_m.to(cuda), noise=inp['noise'].to(cuda))
    assert torch.equal(a, b)
    long_m[:, 100] = True
    with pytest.raises(ValueError):
        m.predict_action(*args, long_t.to(cuda), inp['states'].to(cuda),
                         lang_masks=long_m.to(cuda), noise=inp['noise'].to(cuda))


@pytest.mark.parametrize('h,w,position', [(480, 640, 'center'),
                                          (640, 480, 'top-left'),
                                          (47, 448, 'bottom-right'),
                                          (300, 250, 'top-right'),
                                          (224, 224, 'center')])
def test_letterbox_bit_exact(P, cuda, h, w, position):
    """TransformImage 'letterbox' (the reference's default strategy): Pillow
    resize keeping the aspect ratio, pasted on a per-channel fill colour,
    then (x - mean) / std; every pixel equal to the Pillow restatement in
    uint8, the normalized planes within 1e-5."""
    announce(f'letterbox {h}x{w} {position}')
    src = frames(7, 2, h, w)
    means, stds = (0.5, 0.4, 0.3), (0.5, 0.6, 0.7)
    pre = P.ImagePreprocessor.from_transforms([dict(
        type='TransformImage', image_resize_strategy='letterbox',
        input_sizes=[(3, 224, 224)], means=[means], stds=[stds],
        letterbox_fill=[12, 200, 77], letterbox_pad_position=position)])
    got = pre([src.to(cuda)]).cpu().numpy()
    raw = P.ImagePreprocessor(224, 224, resize='letterbox',
                              pad_value=(12, 200, 77),
                              pad_direction=position)([src.to(cuda)]).cpu()
    for i in range(2):
        ref = PO.transform_image_letterbox(src[i].numpy(), 224, means, stds,
                                           (12, 200, 77), position)
        assert np.abs(got[i] - ref).max() <= 1e-5 * np.abs(ref).max(), i
        ref_u8 = PO.transform_image_letterbox(src[i].numpy(), 224, (0, 0, 0),
                                              (1, 1, 1), (12, 200, 77),
                                              position)
        assert np.array_equal(raw[i].numpy(), ref_u8), i
