"""Host side of the preprocessing before the prefix (CPU): the prompt
tokenizer and padding (fluxvla/tokenizers/paligemma_tokenizer.py:26-75,
fluxvla/transforms/transform_prompts.py:24-110), the parsing of the
reference's transform configs into the fused device preprocessor, and the
pins of the preprocessing oracle (closed forms of the half-pixel bilinear
convention, pad placement, normalization)."""
import io

import numpy as np
import pytest
import torch

from fluxvla_amd import preprocess as P
from oracle import preprocess_oracle as PO

CORPUS = ['pick up the red block and place it in the bowl', 'open the drawer',
          'put the cup on the plate', 'close the door', 'stack the blocks']


@pytest.fixture(scope='module')
def spm_path(tmp_path_factory):
    """A small SentencePiece model trained here (the PaliGemma model file is
    not available offline); BOS id 2 as in PaliGemma's vocabulary."""
    import sentencepiece as spm
    buf = io.BytesIO()
    spm.SentencePieceTrainer.train(
        sentence_iterator=iter(CORPUS * 20), model_writer=buf, vocab_size=40,
        model_type='bpe', bos_id=2, eos_id=1, pad_id=0, unk_id=3,
        user_defined_symbols=['\n'], minloglevel=2)
    path = tmp_path_factory.mktemp('spm') / 'tokenizer.model'
    path.write_bytes(buf.getvalue())
    return str(path)


def test_tokenizer_bos_newline_and_cleaning(spm_path):
    import sentencepiece as spm
    sp = spm.SentencePieceProcessor(model_file=spm_path)
    tok = P.PaligemmaTokenizer(spm_path)
    out = tok('pick up the cup')
    ids = out['input_ids']
    assert ids[0] == sp.bos_id() == 2
    nl = sp.encode('\n')
    assert ids[-len(nl):] == nl
    assert ids[1:-len(nl)] == sp.encode('pick up the cup')
    assert out['attention_mask'] == [True] * len(ids)
    # '_' and newlines become spaces, surrounding blanks are stripped
    assert tok('  pick_up the\ncup \n')['input_ids'] == ids


def test_process_prompts_pads_and_truncates(spm_path):
    tok = P.PaligemmaTokenizer(spm_path)
    n = len(tok('open the drawer')['input_ids'])
    out = P.ProcessPrompts(tok, max_len=n + 5)({'prompt': 'open the drawer'})
    assert out['lang_tokens'].shape == (n + 5,)
    assert list(out['lang_masks']) == [True] * n + [False] * 5
    assert list(out['lang_tokens'][n:]) == [0] * 5
    short = P.ProcessPrompts(tok, max_len=3)({'prompt': 'open the drawer'})
    assert list(short['lang_tokens']) == tok('open the drawer')['input_ids'][:3]
    assert list(short['lang_masks']) == [True] * 3


def test_from_transforms_reference_configs():
    """The PI0 aloha chain and the LIBERO TransformImage chain."""
    means = [[123.515625, 116.04492188, 103.59375]] * 3
    stds = [[58.27148438, 57.02636719, 57.27539062]] * 3
    pre = P.ImagePreprocessor.from_transforms([
        dict(type='ProcessParquetInputs'),
        dict(type='ResizeImages', height=224, width=224),
        dict(type='NormalizeImages', means=means, stds=stds)])
    assert pre.resize == 'linear' and (pre.height, pre.width) == (224, 224)
    m, den = pre._norm(1)
    assert m == tuple(np.float32(means[1]).tolist())
    # numpy: float32 std + 1e-8 stays float32
    assert den == tuple((np.float32(stds[1]) + 1e-8).astype(np.float32).tolist())
    ti = P.ImagePreprocessor.from_transforms([dict(
        type='TransformImage', image_resize_strategy='resize-naive',
        input_sizes=[[3, 224, 224]] * 2, means=means[:2], stds=stds[:2])])
    assert ti.resize == 'pil' and ti._norm(0)[1] == tuple(
        np.float32(stds[0]).tolist())
    # 'letterbox' (the reference's default strategy): fill from the means
    # (int(x * 255)), centred unless letterbox_pad_position says otherwise
    lb = P.ImagePreprocessor.from_transforms([dict(type='TransformImage')])
    assert lb.resize == 'letterbox' and lb.pad_value == (127, 127, 127)
    assert lb.pad_direction == 'center'
    lb2 = P.ImagePreprocessor.from_transforms([dict(
        type='TransformImage', letterbox_fill=[10, 20, 30],
        letterbox_pad_position='top-left')])
    assert lb2.pad_value == (10, 20, 30) and lb2.pad_direction == 'top-left'
    with pytest.raises(ValueError, match='not supported'):
        P.ImagePreprocessor.from_transforms([dict(
            type='TransformImage', image_resize_strategy='squash')])
    with pytest.raises(NotImplementedError):
        P.ImagePreprocessor.from_transforms([dict(
            type='TransformImage', input_sizes=[(3, 224, 256)])])
    pad = P.ImagePreprocessor.from_transforms([dict(
        type='ResizeImagesWithPad', height=224, width=224, pad_value=0,
        pad_direction='top-left')])
    assert pad._region(300, 480) == (84, 0, 140, 224)
    assert P.ImagePreprocessor(224, 224, resize='pad')._region(300, 480) == (
        42, 0, 140, 224)


# ---------------------------------------------------------------------------
# oracle pins
# ---------------------------------------------------------------------------
def test_linear_resize_half_pixel_closed_form():
    """A 4-wide ramp 0, 10, 20, 30 upscaled to 8 samples at half-pixel
    centres: source x = (i + 0.5) / 2 - 0.5 clamped at 0, i.e. 0, 2.5, 7.5,
    ..., 27.5, 30, rounded half up; corner-aligned sampling would give
    0, 4.3, ...; a constant frame stays constant at any size."""
    ramp = np.tile(np.array([0, 10, 20, 30], np.uint8)[None, :, None], (2, 1, 3))
    out = PO.resize_linear_u8(ramp, 2, 8)
    assert out[0, :, 0].tolist() == [0, 3, 8, 13, 18, 23, 28, 30]
    const = np.full((37, 53, 3), 77, np.uint8)
    assert np.all(PO.resize_linear_u8(const, 224, 224) == 77)
    assert np.all(PO.resize_pil_u8(const, 224, 224) == 77)


def test_pil_downscale_averages():
    """Pillow BILINEAR antialiases: a 2x downscale of a 0/100 checkerboard of
    2x2 cells keeps the cell values away from edges, and a 1-pixel
    checkerboard averages to about 50 (a two-tap filter would alias)."""
    cb = (np.indices((64, 64)).sum(0) % 2 * 100).astype(np.uint8)
    img = np.repeat(cb[:, :, None], 3, axis=2)
    out = PO.resize_pil_u8(img, 32, 32).astype(int)
    assert abs(out[8:24, 8:24].mean() - 50) < 2
    assert out[8:24, 8:24].std() < 15


def test_normalize_and_pad_closed_forms():
    img = np.full((1, 3, 2, 2), 200, np.uint8)
    out = PO.normalize_images(img, [[100.0, 50.0, 0.0]], [[50.0, 25.0, 2.0]])
    assert np.allclose(out[0, :, 0, 0], [2.0, 6.0, 100.0])
    unit = PO.normalize_images(img, [[0.5] * 3], [[0.25] * 3],
                               scale_to_unit_interval=True)
    assert np.allclose(unit[0, 0, 0, 0], (200 / 255 - 0.5) / 0.25)
    src = np.full((3, 100, 200), 9, np.uint8)
    padded = PO.resize_chw_with_pad(src, 100, 100, 5, 'bottom-right')
    assert padded.shape == (3, 100, 100)
    assert np.all(padded[:, :50] == 9) and np.all(padded[:, 50:] == 5)
    t = torch.ones(1, 3, 50, 100)
    r = PO.resize_with_pad(t, 224, 224)
    assert r.shape == (1, 3, 224, 224)
    assert torch.all(r[:, :, :112] == -1) and torch.all(r[:, :, 112:] == 1)


def test_letterbox_region_rounds_like_python():
    """letterbox sides are round(side / ratio) (transform_images.py:607-609,
    Python's round: half to even), where ResizeImagesWithPad truncates."""
    lb = P.ImagePreprocessor(224, 224, resize='letterbox')
    assert lb._region(480, 640) == (28, 0, 168, 224)
    # 45 / (448 / 224) = 22.5 -> 22 (half to even); int() also gives 22,
    # 47 / 2 = 23.5 -> 24 where int() gives 23
    assert lb._region(45, 448)[2] == 22
    assert lb._region(47, 448)[2] == 24
    assert P.ImagePreprocessor(224, 224, resize='pad')._region(47, 448)[2] == 23
    corner = P.ImagePreprocessor(224, 224, resize='letterbox',
                                 pad_direction='top-left')
    assert corner._region(47, 448) == (200, 0, 24, 224)


def test_letterbox_oracle_closed_form():
    """A constant frame letterboxed: the picture keeps its value, the rest is
    the fill colour, placed per position; normalization (x - mean) / std in
    0..255 units as the reference does."""
    img = np.full((100, 200, 3), 90, np.uint8)
    out = PO.transform_image_letterbox(img, 64, (0.5, 0.5, 0.5),
                                       (0.5, 0.5, 0.5), (10, 20, 30))
    raw = out * 0.5 + 0.5
    assert np.allclose(raw[:, 16:48, :], 90)
    assert np.allclose(raw[:, :16, :].reshape(3, -1).T, [10, 20, 30])
    assert np.allclose(raw[:, 48:, :].reshape(3, -1).T, [10, 20, 30])
    tl = PO.transform_image_letterbox(img, 64, (0, 0, 0), (1, 1, 1),
                                      (1, 2, 3), 'top-left')
    assert np.allclose(tl[:, 32:, :], 90) and np.allclose(tl[0, :32], 1)
