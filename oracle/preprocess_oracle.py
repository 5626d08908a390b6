"""CPU oracle of the image preprocessing before the prefix.

TEST INFRASTRUCTURE ONLY.  Only tests/ may import this module, and only as
the checker; the product path (fluxvla_amd/preprocess.py) runs the HIP
kernel fvx_resize_normalize and fails loudly without it.

It restates the reference's host transforms with the library routines they
reduce to:

  ResizeImages         fluxvla/transforms/transform_images.py:80-144
                       (cv2.resize INTER_LINEAR on uint8 HWC frames)
  ResizeImagesWithPad  transform_images.py:40-77, 147-189
  NormalizeImages      transform_images.py:313-390
  TransformImage       transform_images.py:414-623, 'resize-naive' and
                       'letterbox' (PIL Image.resize BILINEAR, paste on a
                       fill-colour canvas, (x - mean) / std)
  resize_with_pad      fluxvla/engines/utils/model_utils.py:98-120
                       (F.interpolate bilinear, F.pad left/top)

OpenCV is not installed here, so the cv2 bilinear resize is restated with
torch's bilinear interpolate (align_corners=False, no antialiasing): the
same sampling positions and weights, in floating point, rounded to uint8.
cv2 quantizes its weights to 11 bits, so its uint8 output can differ from
this by one level; that last-bit behaviour is parity unpinned.  Pillow is
installed and is called directly.
"""
import numpy as np
import torch
import torch.nn.functional as F
from PIL import Image


def resize_linear_u8(img_hwc, height, width):
    """uint8 [h, w, 3] -> uint8 [height, width, 3]: bilinear with half-pixel
    centres (cv2.resize INTER_LINEAR), rounded half up and clipped."""
    x = torch.from_numpy(np.ascontiguousarray(img_hwc)).permute(2, 0, 1)
    y = F.interpolate(x[None].float(), size=(height, width), mode='bilinear',
                      align_corners=False)[0]
    y = torch.floor(y + 0.5).clamp(0, 255).to(torch.uint8)
    return y.permute(1, 2, 0).numpy()


def resize_pil_u8(img_hwc, height, width):
    """Image.resize((width, height), BILINEAR) of an RGB uint8 frame."""
    return np.array(Image.fromarray(np.ascontiguousarray(img_hwc)).resize(
        (width, height), Image.Resampling.BILINEAR))


def normalize_images(imgs_chw, means, stds, scale_to_unit_interval=False):
    """NormalizeImages._normalize_flat_images: float32 (x [/ 255] - mean) /
    (std + 1e-8), one (mean, std) row per image."""
    flat = np.asarray(imgs_chw).astype(np.float32)
    if scale_to_unit_interval:
        flat = flat / 255.0
    means = np.asarray(means, dtype=np.float32)
    stds = np.asarray(stds, dtype=np.float32)
    out = [(im - means[i][:, None, None]) / (stds[i][:, None, None] + 1e-8)
           for i, im in enumerate(flat)]
    return np.stack(out, axis=0)


def transform_image_naive(img_hwc, size, mean, std):
    """TransformImage.apply_transform with 'resize-naive': PIL BILINEAR to
    size x size, (x - mean) / std (float64 mean/std), CHW."""
    r = resize_pil_u8(img_hwc, size, size).astype(np.float32)
    out = (r - np.asarray(mean)) / np.asarray(std)
    return out.transpose(2, 0, 1)


def transform_image_letterbox(img_hwc, size, mean, std, fill,
                              position='center'):
    """TransformImage.apply_transform with 'letterbox' at a square size
    (letterbox_pad_transform, transform_images.py:593-623): PIL BILINEAR to
    round(side / ratio) (at least 1), pasted on an RGB canvas of ``fill``
    (centred, or against the corner opposite ``position``'s padding), then
    the resize to size x size (a copy) and (x - mean) / std, CHW."""
    img = Image.fromarray(np.ascontiguousarray(img_hwc))
    ratio = max(img.width / size, img.height / size)
    new_w = max(1, round(img.width / ratio))
    new_h = max(1, round(img.height / ratio))
    img = img.resize((new_w, new_h), Image.Resampling.BILINEAR)
    canvas = Image.new('RGB', (size, size), tuple(fill))
    if position == 'center':
        x0, y0 = (size - img.width) // 2, (size - img.height) // 2
    else:
        x0 = size - img.width if 'left' in position else 0
        y0 = size - img.height if 'top' in position else 0
    canvas.paste(img, (x0, y0))
    r = np.array(canvas.resize((size, size), Image.Resampling.BILINEAR))
    out = (r.astype(np.float32) - np.asarray(mean)) / np.asarray(std)
    return out.transpose(2, 0, 1)


def resize_chw_with_pad(img_chw, height, width, pad_value, pad_direction):
    """_resize_chw_with_pad: aspect-preserving bilinear resize of a uint8
    CHW frame, then constant padding at pad_direction."""
    hwc = np.asarray(img_chw).transpose(1, 2, 0)
    h, w = hwc.shape[:2]
    ratio = max(w / width, h / height)
    rh, rw = max(1, int(h / ratio)), max(1, int(w / ratio))
    r = resize_linear_u8(hwc, rh, rw)
    ph, pw = max(0, height - rh), max(0, width - rw)
    if pad_direction == 'center':
        top, left = ph // 2, pw // 2
        bottom, right = ph - top, pw - left
    else:
        top = ph if 'top' in pad_direction else 0
        bottom = ph if 'bottom' in pad_direction else 0
        left = pw if 'left' in pad_direction else 0
        right = pw if 'right' in pad_direction else 0
    r = np.pad(r, ((top, bottom), (left, right), (0, 0)),
               constant_values=pad_value)
    return r.transpose(2, 0, 1)


def resize_with_pad(img, width, height, pad_value=-1):
    """model_utils.resize_with_pad on a float [b, c, h, w] tensor."""
    cur_h, cur_w = img.shape[2:]
    ratio = max(cur_w / width, cur_h / height)
    rh, rw = int(cur_h / ratio), int(cur_w / ratio)
    r = F.interpolate(img, size=(rh, rw), mode='bilinear',
                      align_corners=False)
    ph, pw = max(0, int(height - rh)), max(0, int(width - rw))
    return F.pad(r, (pw, 0, ph, 0), value=pad_value)
