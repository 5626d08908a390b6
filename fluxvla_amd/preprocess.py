"""The step before the prefix: camera frames and the prompt to model inputs.

Image side: the reference runs its transform chain on the host (numpy, cv2,
PIL) before every request -- ResizeImages + NormalizeImages in the PI0 /
PI0.5 training and serving configs (configs/pi0/pi0_paligemma_aloha_full_
finetune.py:175-183), TransformImage 'resize-naive' in the LIBERO eval
configs (configs/pi05/pi05_paligemma_libero_10_full_inference.py:331-339).
Here one HIP kernel per camera view (fvx_resize_normalize) resizes,
normalizes and reorders the uint8 frames on the GPU, writing straight into
the fp32 [B, 3 * views, H, W] image planes the patch embedding reads.

Prompt side: PaligemmaTokenizer (fluxvla/tokenizers/paligemma_tokenizer.py:
26-75) over a local SentencePiece model, and ProcessPrompts' padding and
truncation (fluxvla/transforms/transform_prompts.py:24-110).  Tokenization
stays on the host: it is a few dozen tokens of string work.
"""
import numpy as np
import torch

from . import kernels as K
from ._lib import RESIZE_LINEAR, RESIZE_PIL_BILINEAR

PAD_POSITIONS = ('top-left', 'top-right', 'bottom-left', 'bottom-right',
                 'center')


def _pad_split(total, direction, first, second):
    """Padding before the picture along one axis (transform_images.py:
    40-75): centered (floor half first), or all before / after."""
    if direction == 'center':
        return total // 2
    if first in direction:
        return total
    return 0


class ImagePreprocessor:
    """A reference image-transform chain fused into one kernel per view.

    resize:
      'linear'   ResizeImages: stretch to height x width with bilinear
                 interpolation (cv2 INTER_LINEAR), rounded to uint8;
      'pad'      ResizeImagesWithPad: keep the aspect ratio (sides
                 int(side / ratio), at least 1), bilinear, pad with
                 pad_value at pad_direction;
      'pil'      TransformImage 'resize-naive' / 'resize-crop': Pillow
                 BILINEAR (antialiased) to height x width;
      'letterbox' TransformImage 'letterbox': Pillow BILINEAR keeping the
                 aspect ratio (sides round(side / ratio), at least 1),
                 pasted at pad_direction onto a canvas of the fill colour
                 pad_value (one raw value per channel, or one for all);
      'none'     the frames already have the target size.
    Normalization per view v and channel c: (x / pre_div - mean[v][c]) /
    den[v][c] -- NormalizeImages: den = std + 1e-8 in fp32, pre_div 255
    with scale_to_unit_interval; TransformImage: den = std.
    """

    def __init__(self, height=224, width=224, resize='linear', means=None,
                 stds=None, eps=1e-8, scale_to_unit_interval=False,
                 pad_value=0, pad_direction='center', swap_rb=False):
        if resize not in ('linear', 'pad', 'pil', 'letterbox', 'none'):
            raise ValueError(f'unknown resize {resize!r}')
        if pad_direction not in PAD_POSITIONS:
            raise ValueError(f"Invalid pad_direction '{pad_direction}'")
        self.height, self.width = height, width
        self.resize = resize
        self.means = None if means is None else np.asarray(means, np.float32)
        self.stds = None if stds is None else np.asarray(stds, np.float32)
        self.eps = eps
        self.pre_div = 255.0 if scale_to_unit_interval else 1.0
        self.pad_value = pad_value
        self.pad_direction = pad_direction
        self.swap_rb = swap_rb

    @classmethod
    def from_transforms(cls, transforms, **kw):
        """Build from a reference transform list (dicts with 'type'); the
        image transforms are fused, the others ignored."""
        args = dict(kw)
        for t in transforms:
            ty = t.get('type')
            if ty == 'ResizeImages':
                args.update(height=t['height'], width=t['width'],
                            resize='linear')
            elif ty == 'ResizeImagesWithPad':
                args.update(height=t['height'], width=t['width'], resize='pad',
                            pad_value=t.get('pad_value', 0),
                            pad_direction=t.get('pad_direction', 'center'))
            elif ty == 'NormalizeImages':
                args.update(means=t['means'], stds=t['stds'],
                            scale_to_unit_interval=t.get(
                                'scale_to_unit_interval', False))
            elif ty == 'TransformImage':
                # transform_images.py:414-623
                strategy = t.get('image_resize_strategy', 'letterbox')
                if strategy not in ('resize-naive', 'resize-crop',
                                    'letterbox'):
                    raise ValueError(f"Image resize strategy '{strategy}' is "
                                     'not supported!')
                size = (t.get('input_sizes') or [(3, 224, 224)])[0]
                if size[-1] != size[-2]:
                    # the reference hands (H, W) to PIL as (width, height)
                    raise NotImplementedError(
                        'TransformImage with non-square input_sizes')
                means = t.get('means') or [(0.5, 0.5, 0.5)]
                args.update(height=size[-2], width=size[-1], resize='pil',
                            means=means,
                            stds=t.get('stds') or [(0.5, 0.5, 0.5)], eps=0.0)
                if strategy == 'letterbox':
                    # one fill for all views, from the last view's means
                    # when none is given (transform_images.py:495-498)
                    fill = t.get('letterbox_fill') or [
                        int(x * 255) for x in means[-1]]
                    args.update(resize='letterbox', pad_value=tuple(fill),
                                pad_direction=t.get('letterbox_pad_position')
                                or 'center')
        return cls(**args)

    def _norm(self, v):
        """(mean, den) of view v in fp32, as numpy computes them."""
        if self.means is None:
            return (0.0, 0.0, 0.0), (1.0, 1.0, 1.0)
        m = self.means if self.means.ndim == 1 else self.means[
            v if self.means.shape[0] > 1 else 0]
        s = self.stds if self.stds.ndim == 1 else self.stds[
            v if self.stds.shape[0] > 1 else 0]
        den = (s + np.float32(self.eps)).astype(np.float32)
        return tuple(float(x) for x in m), tuple(float(x) for x in den)

    def _region(self, h, w):
        H, W = self.height, self.width
        if self.resize not in ('pad', 'letterbox'):
            return 0, 0, H, W
        ratio = max(w / W, h / H)
        if self.resize == 'pad':      # transform_images.py:44-46
            rh, rw = max(1, int(h / ratio)), max(1, int(w / ratio))
        else:                         # :607-609, Python's round
            rh, rw = max(1, round(h / ratio)), max(1, round(w / ratio))
        ph, pw = max(0, H - rh), max(0, W - rw)
        return (_pad_split(ph, self.pad_direction, 'top', 'bottom'),
                _pad_split(pw, self.pad_direction, 'left', 'right'), rh, rw)

    def __call__(self, views, out=None, hwc=True):
        """views: list (one per camera) of uint8 [B, h, w, 3] (hwc) or
        [B, 3, h, w] device tensors.  Returns fp32 [B, 3 * views, H, W]."""
        B = views[0].shape[0]
        if out is None:
            out = torch.empty(B, 3 * len(views), self.height, self.width,
                              dtype=torch.float32, device=views[0].device)
        pil = self.resize in ('pil', 'letterbox')
        for v, img in enumerate(views):
            h, w = (img.shape[1], img.shape[2]) if hwc else img.shape[2:]
            if self.resize == 'none' and (h, w) != (self.height, self.width):
                raise ValueError(f'view {v} is {h}x{w}, expected '
                                 f'{self.height}x{self.width}')
            mean, den = self._norm(v)
            K.resize_normalize(
                img.contiguous(), out[:, 3 * v:3 * v + 3], hwc=hwc,
                region=self._region(h, w), pad_value=self.pad_value,
                filter=(RESIZE_PIL_BILINEAR if pil else RESIZE_LINEAR),
                round_u8=img.dtype == torch.uint8 and not pil,
                swap_rb=self.swap_rb, mean=mean, den=den, pre_div=self.pre_div)
        return out


def resize_with_pad(img, width, height, pad_value=-1):
    """model_utils.resize_with_pad (fluxvla/engines/utils/model_utils.py:
    98-120) on the device: fp32 [b, c, h, w] resized with bilinear
    interpolation (align_corners=False) to (int(h / ratio), int(w / ratio)),
    ratio = max(w / width, h / height), padded on the left and top with
    pad_value."""
    if img.ndim != 4:
        raise ValueError(f'(b, c, h, w) expected, but {img.shape}')
    b, c, h, w = img.shape
    if c != 3:
        raise ValueError('resize_with_pad takes 3-channel images')
    ratio = max(w / width, h / height)
    rh, rw = int(h / ratio), int(w / ratio)
    ph, pw = max(0, int(height - rh)), max(0, int(width - rw))
    out = torch.empty(b, 3, rh + ph, rw + pw, dtype=torch.float32,
                      device=img.device)
    return K.resize_normalize(img.float().contiguous(), out, hwc=False,
                              region=(ph, pw, rh, rw), pad_value=pad_value)


class PaligemmaTokenizer:
    """PaliGemma prompt tokenizer (fluxvla/tokenizers/paligemma_tokenizer.py:
    26-75) over a local SentencePiece model file (the reference downloads
    gs://big_vision/paligemma_tokenizer.model; here the path is given)."""

    def __init__(self, download_path, *args, **kwargs):
        import sentencepiece
        with open(download_path, 'rb') as f:
            self._tokenizer = sentencepiece.SentencePieceProcessor(
                model_proto=f.read())

    def tokenize(self, prompt, state=None, **kwargs):
        """BOS + pieces of the cleaned prompt (stripped, '_' and newlines
        as spaces) + the pieces of '\\n'; all tokens valid."""
        cleaned = prompt.strip().replace('_', ' ').replace('\n', ' ')
        tokens = (self._tokenizer.encode(cleaned, add_bos=True) +
                  self._tokenizer.encode('\n'))
        return dict(input_ids=tokens, attention_mask=[True] * len(tokens))

    def __call__(self, *args, **kwargs):
        return self.tokenize(*args, **kwargs)


class ProcessPrompts:
    """Prompt -> fixed-length lang_tokens / lang_masks
    (transform_prompts.py:24-110): padded with 0 / False to max_len or
    truncated to it."""

    def __init__(self, tokenizer, max_len=180):
        self.tokenizer = tokenizer
        self.max_len = max_len

    def _one(self, prompt, state=None):
        kw = {} if state is None else {'state': state}
        tokens = list(self.tokenizer(prompt, add_special_tokens=True,
                                     **kw)['input_ids'])
        mask = [True] * len(tokens)
        if self.max_len is not None:
            if len(tokens) < self.max_len:
                pad = self.max_len - len(tokens)
                tokens, mask = tokens + [0] * pad, mask + [False] * pad
            else:
                tokens, mask = tokens[:self.max_len], mask[:self.max_len]
        return tokens, mask

    def __call__(self, inputs):
        tokens, mask = self._one(inputs['prompt'], inputs.get('state'))
        inputs['lang_tokens'] = np.array(tokens)
        inputs['lang_masks'] = np.array(mask)
        return inputs
