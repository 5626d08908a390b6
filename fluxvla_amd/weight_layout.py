"""Weight layouts at the drop-in boundary.

The reference's prepare hooks hand its ops weights in the ``[in, out]``
layout (``W.T.contiguous()``: condition_gemma_inference.py:91-105,
siglip_vit_inference.py:41-68, linear_projector_inference.py:8-14), and
``matmul_bias_cuda`` reads ``N = weight.size(1)`` (matmul_bias.py:38-40).
The HIP GEMMs want the reduction dimension contiguous, i.e. ``[out, in]``
(nn.Linear's own layout).  Both are accepted without ambiguity:

* a plain ``torch.Tensor`` always means the reference layout ``[..., in,
  out]``; the ops transpose it once, on first use, and keep the
  ``[out, in]`` copy (keyed by address, shape, strides and version, so an
  in-place update of the weight is seen).  The cache holds the source
  tensor too, so its memory cannot be freed and handed to another tensor
  that would then hit a stale entry; ``clear_layout_cache()`` drops both;
* an ``NKWeight`` -- what this package's prepare hooks emit -- holds the
  ``[..., out, in]`` tensor the kernels read directly.  It presents the
  reference's logical shape ``[..., in, out]`` and indexes like it
  (``w[i]`` is layer i), so code written against the reference's weight
  dicts runs unchanged.

A square weight (SigLIP out_proj 1152 x 1152, Gemma o_proj 2048 x 2048,
the time MLPs 1024 x 1024) can therefore never be applied transposed by
accident: its meaning comes from its type, not its shape.
"""
import torch


class NKWeight:
    """A weight stored ``[..., out, in]`` (K contiguous) standing for the
    reference's ``[..., in, out]`` tensor."""

    __slots__ = ('nk',)

    def __init__(self, nk):
        if not isinstance(nk, torch.Tensor) or nk.dim() < 2:
            raise ValueError('NKWeight wraps a tensor of rank >= 2 '
                             '([..., out, in])')
        self.nk = nk

    @staticmethod
    def from_reference(w_in_out):
        """From a reference-layout tensor [..., in, out] (copied)."""
        return NKWeight(w_in_out.transpose(-1, -2).contiguous())

    # the reference's logical view -------------------------------------------
    @property
    def shape(self):
        s = tuple(self.nk.shape)
        return torch.Size(s[:-2] + (s[-1], s[-2]))

    def size(self, dim=None):
        return self.shape if dim is None else self.shape[dim]

    def dim(self):
        return self.nk.dim()

    @property
    def ndim(self):
        return self.nk.dim()

    @property
    def dtype(self):
        return self.nk.dtype

    @property
    def device(self):
        return self.nk.device

    def __getitem__(self, idx):
        """Index the leading (layer) dimensions only."""
        if self.nk.dim() < 3:
            raise IndexError('an [out, in] NKWeight has no layer dimension '
                             'to index')
        out = self.nk[idx]
        if out.dim() < 2:
            raise IndexError('indexing must keep the two matrix dimensions')
        return NKWeight(out)

    def __len__(self):
        return self.nk.shape[0]

    def to(self, *args, **kwargs):
        return NKWeight(self.nk.to(*args, **kwargs))

    def reference(self):
        """The reference-layout tensor [..., in, out] (a copy)."""
        return self.nk.transpose(-1, -2).contiguous()

    def __repr__(self):
        return (f'NKWeight(logical {tuple(self.shape)} [in, out], stored '
                f'{tuple(self.nk.shape)} [out, in], {self.dtype})')


# [out, in] copies of reference-layout weights, made once per weight and
# kept at one address: key (tag, address, shape, strides, dtype, device) ->
# [source tensor (kept alive so its address stays its own), the source's
# version when the copy was made, the copy, the function that makes it].
# An in-place update of the source (a new version) is copied into the same
# copy tensor, so the cache holds one entry per weight and a HIP graph
# captured over the copy reads the update once the copy is refreshed.
_nk_cache = {}


def clear_layout_cache():
    """Drop the cached [out, in] copies (and the references that keep their
    source weights alive), e.g. after replacing a model's weights.  Graphs
    captured over the dropped copies must be captured again."""
    _nk_cache.clear()


def refresh_layout_cache():
    """Bring every cached copy up to date with an in-place update of its
    source (eager calls do this for the weights they use; call it before
    replaying a graph captured before such an update).  Returns the number
    of copies rewritten."""
    n = 0
    for e in _nk_cache.values():
        if e[0]._version != e[1]:
            e[2].copy_(e[3](e[0]))
            e[1] = e[0]._version
            n += 1
    return n


def _cached(w, tag, make):
    k = (tag, w.data_ptr(), tuple(w.shape), tuple(w.stride()), w.dtype,
         w.device)
    e = _nk_cache.get(k)
    if e is None:
        e = _nk_cache[k] = [w, w._version, make(w), make]
    elif e[1] != w._version:
        e[2].copy_(make(w))
        e[1] = w._version
    return e[2]


def _transpose(w):
    return w.t().contiguous()


def as_nk(w):
    """The ``[out, in]`` tensor the kernels read for weight ``w``: an
    ``NKWeight``'s own tensor, or a reference-layout ``[in, out]`` tensor
    transposed once and cached.  Other prepared weight types (fragment-major
    or fp8 weights from this package's hooks) pass through unchanged."""
    if isinstance(w, NKWeight):
        return w.nk
    if not isinstance(w, torch.Tensor):
        return w
    if w.dim() != 2:
        raise ValueError(f'a reference-layout weight must be [in, out], got '
                         f'shape {tuple(w.shape)}')
    return _cached(w, 'kn', _transpose)


def patch_weight_nk(w, k_pad):
    """Patch-embedding weight as the im2col GEMM reads it: [out, k_pad],
    columns in (channel, ky, kx) order, zero from 3 p p to k_pad.  Accepts
    the reference's [kH, kW, C, out] (siglip_vit_inference.py:20-24, cached
    once) or an ``NKWeight`` already in that layout."""
    if isinstance(w, NKWeight):
        if w.nk.shape[-1] != k_pad:
            raise ValueError(f'patch weight has {w.nk.shape[-1]} columns, '
                             f'the im2col GEMM needs {k_pad}')
        return w.nk
    if w.dim() != 4:
        raise ValueError('a reference patch weight is [kH, kW, C, out], got '
                         f'shape {tuple(w.shape)}')

    def make(src):
        kh, kw, c, n = src.shape
        t = torch.zeros(n, k_pad, dtype=src.dtype, device=src.device)
        t[:, :c * kh * kw] = src.permute(3, 2, 0, 1).reshape(n, c * kh * kw)
        return t
    return _cached(w, f'patch{k_pad}', make)


class PatchWeight(NKWeight):
    """The patch-embedding weight prepared for the im2col GEMM ([out,
    k_pad], (c, ky, kx) columns), presenting the reference's [kH, kW, C,
    out] shape."""

    __slots__ = ('kshape',)

    def __init__(self, nk, kshape):
        super().__init__(nk)
        self.kshape = tuple(kshape)  # (kH, kW, C)

    @property
    def shape(self):
        return torch.Size(self.kshape + (self.nk.shape[0],))

    def reference(self):
        """The reference's [kH, kW, C, out] tensor (a copy)."""
        kh, kw, c = self.kshape
        n = self.nk.shape[0]
        return (self.nk[:, :c * kh * kw].reshape(n, c, kh, kw)
                .permute(2, 3, 1, 0).contiguous())
