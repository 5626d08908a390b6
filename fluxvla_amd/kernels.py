"""Torch-facing wrappers of the C ABI.

Each function takes torch tensors that already live on the GPU, checks dtype,
device and contiguity on the host, builds the C descriptor from raw pointers
and enqueues on ``torch.cuda.current_stream()``.  Nothing here allocates
unless the caller omits an ``out=`` tensor, so calls with preallocated
outputs are safe inside HIP graph capture.
"""
import ctypes

import torch

from . import _lib
from ._lib import AttnDesc, GemmDesc

BF16 = torch.bfloat16

# Split-K / split-KV workspaces (fp32 partials), one pair per device,
# allocated zero-filled before any graph capture.  The GEMM keeps per-tile
# arrival counters in the first 4 KiB of its workspace (zero before the first
# call, left zero by every call), so attention partials go to a buffer of
# their own.  Calls on one stream share them.
WORKSPACE_BYTES = 64 << 20
ATTN_WORKSPACE_BYTES = 32 << 20
_workspaces = {}


def workspace(device=None, kind='gemm'):
    """The per-device ``kind`` ('gemm' or 'attn') workspace."""
    dev = torch.device('cuda', torch.cuda.current_device()
                       if device is None else torch.device(device).index)
    key = (dev.index, kind)
    ws = _workspaces.get(key)
    if ws is None:
        size = WORKSPACE_BYTES if kind == 'gemm' else ATTN_WORKSPACE_BYTES
        ws = torch.zeros(size, dtype=torch.uint8, device=dev)
        _workspaces[key] = ws
    return ws


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _check(t, name, dtype=BF16, contiguous=True, allow_none=False):
    if t is None:
        if allow_none:
            return
        raise ValueError(f'{name} is required')
    if not t.is_cuda:
        raise ValueError(f'{name} must be a CUDA (HIP) tensor')
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f'{name} must be {dtype}, got {t.dtype}')
    if contiguous and not t.is_contiguous():
        raise ValueError(f'{name} must be contiguous')


def _rows_ld(t, name):
    """(rows, leading dim) of a 2-D view with unit column stride (a tensor
    of more dims must be viewable as its rows: evenly spaced)."""
    if t.dim() < 2:
        raise ValueError(f'{name} must be at least 2-D')
    if t.stride(-1) != 1:
        raise ValueError(f'{name} must have unit stride in its last dim')
    if t.dim() == 2:
        return t.shape[0], t.stride(0)
    try:
        t2 = t.view(-1, t.shape[-1])
    except RuntimeError as e:
        raise ValueError(f'{name}: rows are not evenly spaced ({e})') from None
    return t2.shape[0], t2.stride(0)


def _grouped_rows(a):
    """A 3-D ``a`` [groups, rows, k] whose groups are further apart than
    their rows (the action rows behind each sample's state row): (rows,
    group stride in rows) for fvx_gemm_desc.a_row_group, else None."""
    if a.dim() != 3 or a.shape[0] < 2 or a.shape[1] < 1 or a.stride(-1) != 1:
        return None
    g, rs = a.shape[1], a.stride(1)
    if a.stride(0) == g * rs:
        return None
    if rs < a.shape[2] or a.stride(0) % rs or a.stride(0) < g * rs:
        raise ValueError('a: groups of rows must be whole rows apart')
    return g, a.stride(0) // rs


# ---------------------------------------------------------------------------
# Norms
# ---------------------------------------------------------------------------
def rms_norm_residual(x, residual=None, weight=None, eps=1e-6, out=None,
                      residual_out=None):
    """h = x (+ residual); residual_out = bf16(h);
    out = bf16(h * rsqrt(mean(h^2) + eps) * weight).  Returns (out, residual_out)."""
    _check(x, 'x')
    _check(residual, 'residual', allow_none=True)
    _check(weight, 'weight', allow_none=True)
    cols = x.shape[-1]
    rows = x.numel() // cols
    if out is None:
        out = torch.empty_like(x)
    _check(out, 'out')
    if residual_out is not None:
        _check(residual_out, 'residual_out')
    if residual is not None and residual.shape != x.shape:
        raise ValueError('residual must have the shape of x')
    if weight is not None and weight.numel() != cols:
        raise ValueError('weight must have x.shape[-1] elements')
    _lib.call('fvx_rms_norm_residual', _ptr(x), _ptr(residual), _ptr(weight),
              _ptr(out), _ptr(residual_out), rows, cols, float(eps),
              _stream())
    return out, residual_out


def layer_norm(x, weight, bias, eps=1e-6, out=None):
    _check(x, 'x')
    _check(weight, 'weight')
    _check(bias, 'bias')
    cols = x.shape[-1]
    if out is None:
        out = torch.empty_like(x)
    _check(out, 'out')
    _lib.call('fvx_layer_norm', _ptr(x), _ptr(weight), _ptr(bias), _ptr(out),
              x.numel() // cols, cols, float(eps), _stream())
    return out


def adarms_norm(x, style, out=None, gate_out=None, rows_per_style=None,
                eps=1e-6, style_locked=None, lock=None, lock_period=None):
    """style rows [scale | shift | gate] (bf16, 3*cols wide), one per
    ``rows_per_style`` rows of x (default: one style row for all rows).
    ``lock`` (device int32 [1]) with ``style_locked`` (one style row) and
    ``lock_period``: rows with row % lock_period < lock take style_locked
    (the prefix method of real-time chunking)."""
    _check(x, 'x')
    cols = x.shape[-1]
    rows = x.numel() // cols
    _check(style, 'style', contiguous=False)
    srows, sld = _rows_ld(style.view(-1, style.shape[-1]), 'style')
    if rows_per_style is None:
        rows_per_style = max(rows, 1)
    if out is None:
        out = torch.empty_like(x)
    _check(out, 'out')
    _check(gate_out, 'gate_out', allow_none=True)
    if lock is not None:
        _check(lock, 'lock', dtype=torch.int32)
        _check(style_locked, 'style_locked', contiguous=False)
        if style_locked.shape[-1] < 3 * cols:
            raise ValueError('style_locked must hold 3 * cols values')
        _lib.call('fvx_adarms_norm_locked', _ptr(x), _ptr(style),
                  _ptr(style_locked), _ptr(lock), int(lock_period), _ptr(out),
                  _ptr(gate_out), rows, cols, int(rows_per_style), sld,
                  float(eps), _stream())
        return out, gate_out
    _lib.call('fvx_adarms_norm', _ptr(x), _ptr(style), _ptr(out),
              _ptr(gate_out), rows, cols, int(rows_per_style), sld,
              float(eps), _stream())
    return out, gate_out


# ---------------------------------------------------------------------------
# Fragment-major operands (M <= 64 GEMMs): each 16x32 MFMA operand block is
# one contiguous 1 KiB, so the skinny GEMM streams them with fully coalesced
# loads (fvx_gemm_desc.a_frag / b_frag / c_frag).
# ---------------------------------------------------------------------------
class FragA:
    """Activations [m <= 64, k] in the fragment-major layout: a bf16 buffer
    of 64 * k elements, element (r, c) at frag_offset(r, c)."""

    def __init__(self, buf, m, k):
        if m > 64 or k % 32 or buf.numel() < 64 * k:
            raise ValueError(f'FragA needs m <= 64, k % 32 == 0 and 64*k '
                             f'elements (m={m}, k={k}, numel={buf.numel()})')
        self.buf, self.m, self.k = buf, m, k

    @staticmethod
    def empty(k, device):
        return FragA(torch.zeros(64 * k, dtype=BF16, device=device), 64, k)

    def rows(self, m):
        return FragA(self.buf, m, self.k)


class FragB:
    """A weight [n, k] (nn.Linear layout) in the fragment-major layout
    [n/16][k/32][4][16][8]; n % 16 == 0, k % 32 == 0."""

    def __init__(self, buf, n, k):
        self.buf, self.n, self.k = buf, n, k

    @staticmethod
    def pack(w):
        n, k = w.shape
        if n % 16 or k % 32:
            raise ValueError(f'FragB needs n % 16 == 0 and k % 32 == 0, got '
                             f'{tuple(w.shape)}')
        buf = (w.reshape(n // 16, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4)
               .contiguous().view(-1))
        return FragB(buf, n, k)


FP8_ACTS = ('bf16', 'e4m3')


class Fp8Weight:
    """An nn.Linear weight [n, k] quantized to OCP e4m3fn (max 448) with one
    fp32 scale per output channel: W[j] ~= scale[j] * e4m3(data[j]),
    scale[j] = max_i |W[j, i]| / 448.  ``data`` is uint8, row-major
    ([n, k], ldb = k bytes) or, with ``frag``, in the fp8 fragment-major
    layout of fvx_gemm_desc (one 16 x 128 MFMA operand per 2 KiB; needs
    n % 16 == 0 and k % 128 == 0) for the M <= 64 skinny GEMM.

    ``act`` selects the GEMM arithmetic (fvx_gemm_desc.fp8_act): 'bf16'
    (W8A16, the default: the e4m3 bytes become bf16 in registers, bf16
    MFMA, fp32 accumulation, i.e. exactly a @ dequantize()^T) or 'e4m3'
    (W8A8: the activations are quantized to e4m3 per row and k step)."""

    def __init__(self, data, scale, n, k, frag=False, act='bf16'):
        if act not in FP8_ACTS:
            raise ValueError(f'act must be one of {FP8_ACTS}, got {act!r}')
        self.data, self.scale, self.n, self.k, self.frag = data, scale, n, k, frag
        self.act = act

    @staticmethod
    def quantize(w, act='bf16'):
        n, k = w.shape
        wf = w.float()
        s = (wf.abs().amax(1) / 448.0).clamp_min(torch.finfo(torch.float32).tiny)
        q = (wf / s[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
        return Fp8Weight(q.contiguous(), s.contiguous(), n, k, act=act)

    def dequantize(self):
        """fp32 [n, k] (row-major weights only)."""
        if self.frag:
            raise ValueError('dequantize needs the row-major layout')
        return (self.data.view(torch.float8_e4m3fn).float() *
                self.scale[:, None])

    def rows(self, start, end=None):
        """Output channels [start, end) (row-major weights only)."""
        if self.frag:
            raise ValueError('rows() needs the row-major layout')
        end = self.n if end is None else end
        return Fp8Weight(self.data[start:end], self.scale[start:end],
                         end - start, self.k, act=self.act)

    def pack_frag(self):
        """Fragment-major copy: byte (n, k) of block (n/16, k/128) at lane
        16 g + n%16, position 8 t + j, where k%128 = 32 t + 8 g + j."""
        n, k = self.n, self.k
        if n % 16 or k % 128:
            raise ValueError(f'fp8 fragment-major weights need n % 16 == 0 '
                             f'and k % 128 == 0, got {(n, k)}')
        buf = (self.data.view(n // 16, 16, k // 128, 4, 4, 8)
               .permute(0, 2, 4, 1, 3, 5).contiguous().view(-1))
        return Fp8Weight(buf, self.scale, n, k, frag=True, act=self.act)


class Fp8Act:
    """An e4m3 copy of an activation matrix [m, k] written by the GEMM that
    produced it (``gemm(..., a8_out=)``) and read as A by the fp8-weight
    wide GEMM (``a8=``): ``data`` uint8 [m, k], ``scale`` uint8 E8M0
    exponents [k / 64, m] (one per row and 64-column block)."""

    def __init__(self, data, scale):
        self.data, self.scale = data, scale

    @staticmethod
    def empty(m, k, device):
        if k % 64:
            raise ValueError('Fp8Act needs k % 64 == 0')
        m4 = (m + 3) // 4 * 4
        return Fp8Act(torch.zeros(m, k, dtype=torch.uint8, device=device),
                      torch.zeros(k // 64, m4, dtype=torch.uint8, device=device))

    def values(self):
        """fp32 values it stands for (dequantized)."""
        m, k = self.data.shape
        q = self.data.view(torch.float8_e4m3fn).float()
        e = self.scale[:, :m].t().float()                     # [m, k / 64]
        return q * torch.pow(2.0, e - 127.0).repeat_interleave(64, 1)


def pack_frag_a_ref(a):
    """Torch restatement of the FragA layout (tests): [m <= 64, k] ->
    64 * k elements; rows >= m are zero."""
    m, k = a.shape
    full = torch.zeros(64, k, dtype=a.dtype, device=a.device)
    full[:m] = a
    return (full.view(4, 16, k // 32, 4, 8).permute(2, 0, 3, 1, 4)
            .contiguous().view(-1))


def pack_frag(src, dst):
    """Row-major [m <= 64, k] -> FragA ``dst`` (device kernel)."""
    _check(src, 'src', contiguous=False)
    rows, sld = _rows_ld(src, 'src')
    _check(dst.buf, 'dst')
    if dst.k != src.shape[-1]:
        raise ValueError('pack_frag: k mismatch')
    _lib.call('fvx_pack_frag', _ptr(src), sld, _ptr(dst.buf), rows,
              src.shape[-1], _stream())
    return dst


# ---------------------------------------------------------------------------
# GEMM family
# ---------------------------------------------------------------------------
def _gemm_desc(a, w):
    d = GemmDesc()
    if isinstance(a, FragA):
        _check(a.buf, 'a')
        m, lda, k = a.m, a.k, a.k
        d.a, d.a_frag, dev = a.buf.data_ptr(), 1, a.buf.device
    else:
        _check(a, 'a', contiguous=False)
        grp = _grouped_rows(a)
        if grp is not None:
            m, lda = a.shape[0] * a.shape[1], a.stride(1)
            d.a_row_group, d.a_row_group_stride = grp
        else:
            m, lda = _rows_ld(a, 'a')
        k = a.shape[-1]
        d.a, dev = a.data_ptr(), a.device
    if isinstance(w, FragB):
        _check(w.buf, 'weight')
        n, ldb, kw = w.n, w.k, w.k
        d.b, d.b_frag = w.buf.data_ptr(), 1
    elif isinstance(w, Fp8Weight):
        _check(w.data, 'weight', dtype=torch.uint8, contiguous=not w.frag)
        _check(w.scale, 'weight scale', dtype=torch.float32)
        n, kw = w.n, w.k
        ldb = w.k if w.frag else w.data.stride(0)
        d.b, d.b_frag, d.b_fp8 = w.data.data_ptr(), int(w.frag), 1
        d.b_scale = w.scale.data_ptr()
        d.fp8_act = int(w.act == 'e4m3')
    else:
        _check(w, 'weight', contiguous=False)
        n, ldb = _rows_ld(w, 'weight')
        kw = w.shape[-1]
        d.b = w.data_ptr()
    if kw != k:
        raise ValueError(
            f'weight must be [out_features, in_features={k}] (nn.Linear '
            f'layout), got in_features={kw}')
    d.lda, d.ldb = lda, ldb
    d.m, d.n, d.k = m, n, k
    d.gate_group = 1
    ws = workspace(dev)
    d.workspace, d.workspace_bytes = ws.data_ptr(), ws.numel()
    return d


def fvx_workspace_bytes(d):
    """Split-K workspace bytes fvx_gemm would use for descriptor ``d``."""
    return _lib.load().fvx_gemm_workspace_bytes(ctypes.byref(d))


def _lead_shape(a):
    return (a.m,) if isinstance(a, FragA) else tuple(a.shape[:-1])


def _device(a):
    return a.buf.device if isinstance(a, FragA) else a.device


def _set_c_frag(d, c_frag):
    if c_frag is not None:
        if c_frag.k != d.n:
            raise ValueError('c_frag must have k == n of the GEMM')
        _check(c_frag.buf, 'c_frag')
        d.c_frag = c_frag.buf.data_ptr()


def _run_gemm(d, noalloc=False):
    if noalloc:
        # library-owned static scratch instead of the caller's workspace
        d.workspace, d.workspace_bytes = None, 0
        _lib.call('fvx_gemm_noalloc', ctypes.byref(d), _stream())
    else:
        _lib.call('fvx_gemm', ctypes.byref(d), _stream())


def ss_parts(n):
    """Parts of the row sums of squares a GEMM with n output columns hands
    over (one per 64-column block)."""
    return (n + 63) // 64


def _set_a8(d, a8=None, a8_out=None):
    """e4m3 activation hand-over (see Fp8Act)."""
    if a8_out is not None:
        _check(a8_out.data, 'a8_out', dtype=torch.uint8)
        _check(a8_out.scale, 'a8_out scale', dtype=torch.uint8)
        if a8_out.data.shape[0] < d.m or a8_out.data.shape[1] < d.n:
            raise ValueError('a8_out is smaller than the output')
        d.a8_out, d.a8_out_ld = a8_out.data.data_ptr(), a8_out.data.stride(0)
        d.a8_out_scale, d.a8_out_sld = a8_out.scale.data_ptr(), a8_out.scale.stride(0)
    if a8 is not None:
        _check(a8.data, 'a8', dtype=torch.uint8)
        _check(a8.scale, 'a8 scale', dtype=torch.uint8)
        if a8.data.shape[0] < d.m or a8.data.shape[1] < d.k:
            raise ValueError('a8 is smaller than A')
        d.a8, d.a8_ld = a8.data.data_ptr(), a8.data.stride(0)
        d.a8_scale, d.a8_sld = a8.scale.data_ptr(), a8.scale.stride(0)


def _set_ss(d, rownorm_eps, ss_in=None, ss_out=None, ln_csum=None):
    """Row sums of squares handed between GEMMs: ``ss_out`` (fp32 [parts,
    ld], parts = ss_parts(n)) receives the producer's per-block sums of its
    squared bf16 outputs; ``ss_in`` (same layout, from the GEMM that wrote
    this GEMM's A) replaces the fused RMSNorm's pass over A.  ``ln_csum``
    (fp32 [N], the weight's column sums): the fused norm is a LayerNorm on
    row sums of A's values and squares taken in the K loop
    (fvx_gemm_desc.ln_csum)."""
    if rownorm_eps is not None:
        d.rownorm, d.rownorm_eps = 1, float(rownorm_eps)
    if ss_in is not None:
        if rownorm_eps is None:
            raise ValueError('ss_in needs rownorm_eps')
        _check(ss_in, 'ss_in', dtype=torch.float32, contiguous=False)
        if ss_in.dim() != 2 or ss_in.stride(1) != 1 or ss_in.shape[1] < d.m:
            raise ValueError('ss_in must be [parts, >= m] with unit row stride')
        d.ss_in, d.ss_parts, d.ss_ld = ss_in.data_ptr(), ss_in.shape[0], ss_in.stride(0)
    if ss_out is not None:
        _check(ss_out, 'ss_out', dtype=torch.float32, contiguous=False)
        if (ss_out.dim() != 2 or ss_out.stride(1) != 1 or ss_out.shape[1] < d.m or
                ss_out.shape[0] < ss_parts(d.n)):
            raise ValueError(f'ss_out must be [>= {ss_parts(d.n)}, >= m] with unit row stride')
        if ss_in is not None and ss_out.stride(0) != d.ss_ld:
            raise ValueError('ss_in and ss_out need the same row stride (one ss_ld)')
        d.ss_out, d.ss_ld = ss_out.data_ptr(), ss_out.stride(0)
    if ln_csum is not None:
        _check(ln_csum, 'ln_csum', dtype=torch.float32)
        if ln_csum.numel() < d.n or rownorm_eps is None or ss_in is not None:
            raise ValueError('ln_csum needs N values and rownorm_eps, and takes no ss_in')
        d.ln_csum = ln_csum.data_ptr()


def gemm(a, weight, out=None, *, bias=None, bias_f32=None, residual=None,
         gate=None, gate_group=1, pos=None, pos_period=0, act=_lib.ACT_NONE,
         rownorm_eps=None, out_f32=False, row_group=0, row_group_stride=0,
         split_k=0, c_frag=None, ss_in=None, ss_out=None, a8=None, a8_out=None,
         noalloc=False, rtc_lock=None, rtc_period=0, bias_f32_locked=None,
         ln_csum=None):
    """out = epilogue(a @ weight^T); see fvx_gemm_desc for the order.
    ``a`` may be a FragA and ``weight`` a FragB; ``c_frag`` (a FragA with
    k == n) also receives the output in the fragment-major layout;
    ``ss_in`` / ``ss_out`` / ``ln_csum``: see _set_ss; ``a8`` / ``a8_out``:
    see Fp8Act.
    ``noalloc``: run through fvx_gemm_noalloc (split-K scratch in the
    library's static device array, no workspace).  ``rtc_lock`` (device
    int32 [1]), ``rtc_period``, ``bias_f32_locked``: rows with
    m % rtc_period < rtc_lock add bias_f32_locked instead of bias_f32."""
    d = _gemm_desc(a, weight)
    if out is None:
        out = torch.empty(*_lead_shape(a), d.n,
                          dtype=torch.float32 if out_f32 else BF16,
                          device=_device(a))
    _check(out, 'out', dtype=torch.float32 if out_f32 else BF16,
           contiguous=False)
    _, d.ldc = _rows_ld(out, 'out')
    d.c = out.data_ptr()
    if bias is not None:
        _check(bias, 'bias')
        d.bias = bias.data_ptr()
    if bias_f32 is not None:
        _check(bias_f32, 'bias_f32', dtype=torch.float32)
        d.bias_f32 = bias_f32.data_ptr()
    if residual is not None:
        _check(residual, 'residual', contiguous=False)
        _, d.ldr = _rows_ld(residual, 'residual')
        d.residual = residual.data_ptr()
    if gate is not None:
        _check(gate, 'gate', contiguous=False)
        _, d.ldg = _rows_ld(gate, 'gate')
        d.gate, d.gate_group = gate.data_ptr(), gate_group
    if pos is not None:
        _check(pos, 'pos', contiguous=False)
        _, d.ldp = _rows_ld(pos, 'pos')
        d.pos, d.pos_period = pos.data_ptr(), pos_period or pos.shape[0]
    d.act, d.mode, d.out_f32 = int(act), _lib.GEMM_PLAIN, int(bool(out_f32))
    _set_rtc(d, rtc_lock, rtc_period, bias_f32_locked)
    _set_ss(d, rownorm_eps, ss_in, ss_out, ln_csum)
    _set_a8(d, a8, a8_out)
    d.row_group, d.row_group_stride = row_group, row_group_stride
    d.split_k = split_k
    _set_c_frag(d, c_frag)
    _run_gemm(d, noalloc)
    return out


def _set_a_scale(d, a_scale=None, bias_f32=None, bias2_f32=None):
    """Adaptive RMSNorm folded into an M <= 64 GEMM (fvx_gemm_desc.a_scale):
    A's column k times (1 + a_scale[k]) (bf16 [K]: the style's scale); fp32
    biases after the RMS factor (QKV_ROPE: bias_f32; GEGLU: bias_f32 gate
    half, bias2_f32 up)."""
    if a_scale is not None:
        _check(a_scale, 'a_scale')
        if a_scale.numel() < d.k:
            raise ValueError('a_scale needs K values')
        d.a_scale = a_scale.data_ptr()
    for t, nm in ((bias_f32, 'bias_f32'), (bias2_f32, 'bias2_f32')):
        if t is not None:
            _check(t, nm, dtype=torch.float32)
            if t.numel() < d.n:
                raise ValueError(f'{nm} needs N values')
            setattr(d, nm, t.data_ptr())


def gemm_geglu(a, gate_w, up_w, out=None, rownorm_eps=None, split_k=0,
               c_frag=None, ss_in=None, a8=None, a8_out=None, a_scale=None,
               bias_f32=None, bias2_f32=None, gu_out=None):
    """out = gelu_tanh(a @ gate_w^T) * (a @ up_w^T); with ``a_scale`` (the
    folded adaptive RMSNorm, M <= 64): gelu_tanh(r a' @ gate_w^T + bias_f32)
    * (r a' @ up_w^T + bias2_f32), a' = a * (1 + a_scale), r the RMS factor
    of a.  ``gu_out`` (bf16 [M, 2N] view): the gate and up values the
    product is taken from (fvx_gemm_desc.gu_out)."""
    d = _gemm_desc(a, gate_w)
    if isinstance(gate_w, Fp8Weight):
        if (not isinstance(up_w, Fp8Weight) or up_w.frag != gate_w.frag or
                up_w.act != gate_w.act or
                (up_w.n, up_w.k) != (gate_w.n, gate_w.k) or
                (not up_w.frag and up_w.data.stride() != gate_w.data.stride())):
            raise ValueError('up_w must be an Fp8Weight laid out like gate_w')
        _check(up_w.scale, 'up_w scale', dtype=torch.float32)
        d.b2, d.b2_scale = up_w.data.data_ptr(), up_w.scale.data_ptr()
    elif isinstance(gate_w, FragB):
        if not isinstance(up_w, FragB) or (up_w.n, up_w.k) != (gate_w.n, gate_w.k):
            raise ValueError('up_w must be a FragB shaped like gate_w')
        _check(up_w.buf, 'up_w')
        d.b2 = up_w.buf.data_ptr()
    else:
        _check(up_w, 'up_w', contiguous=False)
        if tuple(up_w.shape) != tuple(gate_w.shape) or up_w.stride() != gate_w.stride():
            raise ValueError('up_w must match gate_w in shape and strides')
        d.b2 = up_w.data_ptr()
    if out is None:
        out = torch.empty(*_lead_shape(a), d.n, dtype=BF16, device=_device(a))
    _check(out, 'out', contiguous=False)
    _, d.ldc = _rows_ld(out, 'out')
    d.c, d.mode = out.data_ptr(), _lib.GEMM_GEGLU
    _set_a_scale(d, a_scale, bias_f32, bias2_f32)
    _set_ss(d, rownorm_eps, ss_in)
    _set_a8(d, a8, a8_out)
    d.split_k = split_k
    _set_c_frag(d, c_frag)
    if gu_out is not None:
        _check(gu_out, 'gu_out', contiguous=False)
        rows, d.ld_gu = _rows_ld(gu_out, 'gu_out')
        if gu_out.shape[-1] != 2 * d.n or rows != d.m:
            raise ValueError(f'gu_out must be [{d.m}, {2 * d.n}]')
        d.gu_out = gu_out.data_ptr()
    _run_gemm(d)
    return out


def gemm_qkv_rope(a, w_qkv, rope, positions, q_out, k_out, v_out, n_q_heads,
                  head_dim, rownorm_eps=None, row_group=0, row_group_stride=0,
                  split_k=0, v_ld=None, ss_in=None, a8=None, a_scale=None,
                  bias_f32=None, k_t_out=None, kt_ld=None, v_rows_out=None):
    """[q|k|v] = a @ w_qkv^T with pair-interleaved RoPE on q and k.

    rope: fp32 [max_pos, head_dim/2, 2] (cos, sin); positions: int32 [M].
    k_out rows are remapped with (row_group, row_group_stride).  v_out is
    row-major like k_out, or -- with ``v_ld`` given -- the transposed value
    cache: element (m, d) at v_out[(m // row_group * head_dim + d) * v_ld +
    m % row_group] (v_out may be a view offset to the first token column).
    With a transposed v_out, ``k_t_out`` (+ ``kt_ld``) also receives the
    keys transposed the same way and ``v_rows_out`` the values row-major
    with k_out's rows (fvx_gemm_desc.k_t_out / v_rows_out)."""
    d = _gemm_desc(a, w_qkv)
    _check(rope, 'rope', dtype=torch.float32)
    _check(positions, 'positions', dtype=torch.int32)
    if positions.numel() < d.m:
        raise ValueError('positions must have one entry per row of a')
    for t, nm in ((q_out, 'q_out'), (k_out, 'k_out'), (v_out, 'v_out')):
        _check(t, nm, contiguous=False)
    d.mode = _lib.GEMM_QKV_ROPE
    d.rope, d.positions = rope.data_ptr(), positions.data_ptr()
    d.q_out, d.ldq = q_out.data_ptr(), _rows_ld(q_out, 'q_out')[1]
    d.k_out, d.ldk = k_out.data_ptr(), _rows_ld(k_out, 'k_out')[1]
    if v_ld is None:
        d.v_out, d.ldv = v_out.data_ptr(), _rows_ld(v_out, 'v_out')[1]
    else:
        d.v_out, d.ldv, d.v_transposed = v_out.data_ptr(), int(v_ld), 1
    if k_t_out is not None:
        _check(k_t_out, 'k_t_out', contiguous=False)
        d.k_t_out, d.ld_kt = k_t_out.data_ptr(), int(kt_ld)
    if v_rows_out is not None:
        _check(v_rows_out, 'v_rows_out', contiguous=False)
        d.v_rows_out, d.ld_vr = v_rows_out.data_ptr(), _rows_ld(v_rows_out, 'v_rows_out')[1]
    d.n_q_heads, d.head_dim = n_q_heads, head_dim
    _set_a_scale(d, a_scale, bias_f32)
    _set_ss(d, rownorm_eps, ss_in)
    _set_a8(d, a8)
    d.row_group, d.row_group_stride = row_group, row_group_stride
    d.split_k = split_k
    _run_gemm(d)


def _set_rtc(d, lock=None, period=0, bias_f32_locked=None, prev=None,
             cw=None, omt=0.0):
    """Real-time chunking fields of fvx_gemm_desc (rtc_*)."""
    if lock is None and bias_f32_locked is None and prev is None and cw is None:
        return
    if period <= 0:
        raise ValueError('real-time chunking needs rtc_period > 0')
    d.rtc_period = int(period)
    if lock is not None:
        _check(lock, 'rtc_lock', dtype=torch.int32)
        d.rtc_lock = lock.data_ptr()
    if bias_f32_locked is not None:
        _check(bias_f32_locked, 'bias_f32_locked', dtype=torch.float32)
        if bias_f32_locked.numel() < d.n:
            raise ValueError('bias_f32_locked needs n values')
        d.bias_f32_locked = bias_f32_locked.data_ptr()
    if prev is not None:
        _check(prev, 'rtc_prev', dtype=torch.float32, contiguous=False)
        rows, d.ld_prev = _rows_ld(prev, 'rtc_prev')
        if rows < d.m or prev.shape[-1] < d.n:
            raise ValueError(f'rtc_prev must cover [{d.m}, {d.n}]')
        d.rtc_prev = prev.data_ptr()
    if cw is not None:
        _check(cw, 'rtc_cw', dtype=torch.float32)
        if cw.numel() < period:
            raise ValueError('rtc_cw needs rtc_period values')
        d.rtc_cw, d.rtc_omt = cw.data_ptr(), float(omt)


def gemm_euler(a, weight, bias, xt, dt, xt_bf16=None, rownorm_eps=None,
               split_k=0, bias_f32=None, rtc_lock=None, rtc_period=0,
               rtc_prev=None, rtc_cw=None, rtc_omt=0.0, a_scale=None):
    """v = a @ weight^T + bias; xt += dt * v (fp32, in place); xt_bf16 mirrors.
    Real-time chunking (see fvx_gemm_desc): rows with m % rtc_period <
    rtc_lock store rtc_prev (prefix method); with ``rtc_cw`` every row adds
    rtc_cw[m % rtc_period] * (rtc_prev - xt + rtc_omt * v) (guidance)."""
    d = _gemm_desc(a, weight)
    _check(xt, 'xt', dtype=torch.float32, contiguous=False)
    d.mode = _lib.GEMM_EULER
    d.xt, d.ldx = xt.data_ptr(), _rows_ld(xt, 'xt')[1]
    if xt_bf16 is not None:
        _check(xt_bf16, 'xt_bf16', contiguous=False)
        d.xt_bf16, d.ldxb = xt_bf16.data_ptr(), _rows_ld(xt_bf16, 'xt_bf16')[1]
    if bias is not None:
        _check(bias, 'bias')
        d.bias = bias.data_ptr()
    if bias_f32 is not None:
        _check(bias_f32, 'bias_f32', dtype=torch.float32)
        d.bias_f32 = bias_f32.data_ptr()
    d.dt = float(dt)
    if rownorm_eps is not None:
        d.rownorm, d.rownorm_eps = 1, float(rownorm_eps)
    _set_rtc(d, rtc_lock, rtc_period, prev=rtc_prev, cw=rtc_cw, omt=rtc_omt)
    _set_a_scale(d, a_scale)
    d.split_k = split_k
    _run_gemm(d)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
def attention_desc(q, k, v, o, *, sq, sk, heads, head_dim, n_problems=1,
                   zdiv=1, q_tok_stride, q_head_stride, q_zs=(0, 0),
                   k_tok_stride, k_zs=(0, 0), v_tok_stride, v_zs=(0, 0),
                   o_tok_stride, o_head_stride, o_zs=(0, 0), kgrp=None,
                   qgrp=None, kgrp_zs=0, qgrp_zs=0, scale=None, kv_splits=0,
                   v_d_stride=0):
    for t, nm in ((q, 'q'), (k, 'k'), (v, 'v'), (o, 'o')):
        _check(t, nm, contiguous=False)
    d = AttnDesc()
    d.q, d.q_tok_stride, d.q_head_stride = q.data_ptr(), q_tok_stride, q_head_stride
    d.q_zs1, d.q_zs2 = q_zs
    d.k, d.k_tok_stride = k.data_ptr(), k_tok_stride
    d.k_zs1, d.k_zs2 = k_zs
    d.v, d.v_tok_stride = v.data_ptr(), v_tok_stride
    d.v_zs1, d.v_zs2 = v_zs
    d.v_d_stride = v_d_stride
    d.o, d.o_tok_stride, d.o_head_stride = o.data_ptr(), o_tok_stride, o_head_stride
    d.o_zs1, d.o_zs2 = o_zs
    if (kgrp is None) != (qgrp is None):
        raise ValueError('kgrp and qgrp must be given together')
    if kgrp is not None:
        _check(kgrp, 'kgrp', dtype=torch.int32, contiguous=False)
        _check(qgrp, 'qgrp', dtype=torch.int32, contiguous=False)
        if kgrp.stride(-1) != 1 or qgrp.stride(-1) != 1:
            raise ValueError('kgrp and qgrp need unit stride along tokens')
        d.kgrp, d.qgrp = kgrp.data_ptr(), qgrp.data_ptr()
        d.kgrp_zs1, d.qgrp_zs1 = kgrp_zs, qgrp_zs
    d.sq, d.sk, d.heads, d.head_dim = sq, sk, heads, head_dim
    d.n_problems, d.zdiv = n_problems, zdiv
    d.scale = float(head_dim ** -0.5 if scale is None else scale)
    d.kv_splits = kv_splits
    ws = workspace(q.device, 'attn')
    d.workspace, d.workspace_bytes = ws.data_ptr(), ws.numel()
    return d


def run_attention(d):
    _lib.call('fvx_attention', ctypes.byref(d), _stream())


def attention_check(device=None):
    """Raise FvxError (status FVX_ERR_MERGE) when an in-launch merge of the
    decode attention on ``device`` stopped waiting for its key ranges since
    the last check; the merge counters are then cleared, so the next call is
    correct.  Waits for the current stream: call it after a call or a chunk,
    never under graph capture."""
    ws = workspace(device, 'attn')
    _lib.call('fvx_attention_check', ctypes.c_void_p(ws.data_ptr()),
              ctypes.c_int64(ws.numel()), _stream())


def _device_buffer(t):
    """The device tensor behind a weight object (fragment-major, fp8 or
    plain)."""
    if isinstance(t, FragB):
        return t.buf
    if isinstance(t, Fp8Weight):
        return t.data
    return t


def _set_prefetch(d, prefetch, prefetch_wgs, place=True):
    """Up to 8 ranges the decode attention's idle workgroups pull into the
    caches (fvx_attn_desc.prefetch).  Fragment-major weights (FragB, frag
    Fp8Weight) are sequences of 16-column tiles, tile j read by a workgroup
    on XCD j % 8: with ``place`` each tile is fetched from that XCD."""
    items = list(prefetch or ())
    if len(items) > 8:
        raise ValueError('at most 8 prefetch ranges')
    for i, t in enumerate(items):
        buf = _device_buffer(t)
        _check(buf, f'prefetch[{i}]', dtype=None)
        nbytes = buf.numel() * buf.element_size()
        tile = 0
        if place and (isinstance(t, FragB) or
                      (isinstance(t, Fp8Weight) and t.frag)):
            tile = nbytes // (t.n // 16)
            if tile % 1024:
                tile = 0
        d.prefetch[i] = buf.data_ptr()
        d.prefetch_bytes[i] = nbytes - nbytes % 1024
        d.prefetch_tile_bytes[i] = tile
    d.prefetch_wgs = int(prefetch_wgs)


def mqa_attention(q, k, v, o, kgrp=None, qgrp=None, scale=None, kv_splits=0,
                  v_transposed=False, o_frag=None, prefetch=None,
                  prefetch_wgs=0, prefetch_place=True, merge_no_wait=False,
                  o_row_major=True):
    """Batched multi-query attention.

    q: [B, Sq, H, D] (or [B, Sq, H*D]); k: [B, Sk, D] (row stride may exceed
    D, e.g. a cache slice); v: [B, Sk, D], or with ``v_transposed`` the value
    cache [B, D, T >= Sk] (keys contiguous); o like q.  kgrp: int32 [B, Sk],
    qgrp: int32 [B, Sq] (visible iff kgrp[j] <= qgrp[i]).  ``o_frag`` (a
    FragA with k = H*D, decode path only) also receives the output in the
    fragment-major layout, ready as the o-projection's A operand; with
    ``o_row_major=False`` only that copy is written (``o`` then only gives
    the shape).
    ``prefetch``: up to 8 tensors / prepared weights that idle workgroups
    of the decode kernel read into the caches meanwhile (the next GEMMs'
    weights; ``prefetch_wgs`` of them, 0 = fill the CUs; see
    _set_prefetch for ``prefetch_place``).  ``merge_no_wait`` is a test
    hook: the in-launch merge gives up its wait at once (attention_check
    then reports it)."""
    B, Sq = q.shape[0], q.shape[1]
    D = k.shape[-1]
    H = (q.shape[2] if q.dim() == 4 else q.shape[2] // D)
    Sk = k.shape[1]
    if v_transposed and (v.shape[1] != D or v.stride(2) != 1):
        raise ValueError('transposed v must be [B, D, T] with unit key stride')
    d = attention_desc(
        q, k, v, o, sq=Sq, sk=Sk, heads=H, head_dim=D, n_problems=B, zdiv=1,
        q_tok_stride=q.stride(1), q_head_stride=D, q_zs=(q.stride(0), 0),
        k_tok_stride=k.stride(1), k_zs=(k.stride(0), 0),
        v_tok_stride=0 if v_transposed else v.stride(1),
        v_zs=(v.stride(0), 0),
        v_d_stride=v.stride(1) if v_transposed else 0,
        o_tok_stride=o.stride(1), o_head_stride=D, o_zs=(o.stride(0), 0),
        kgrp=kgrp, qgrp=qgrp,
        kgrp_zs=(kgrp.stride(0) if kgrp is not None else 0),
        qgrp_zs=(qgrp.stride(0) if qgrp is not None else 0), scale=scale,
        kv_splits=kv_splits)
    if o_frag is not None:
        if o_frag.k != H * D:
            raise ValueError('o_frag must have k == heads * head_dim')
        _check(o_frag.buf, 'o_frag')
        d.o_frag = o_frag.buf.data_ptr()
    if prefetch:
        _set_prefetch(d, prefetch, prefetch_wgs, prefetch_place)
    d.merge_no_wait = int(bool(merge_no_wait))
    if not o_row_major:
        if o_frag is None:
            raise ValueError('o_row_major=False needs o_frag')
        d.o = None
    run_attention(d)
    return o


def mha_packed_qkv(qkv, out, n_views, seq, heads, head_dim, scale=None,
                   kv_splits=0):
    """Bidirectional MHA over packed [n_views * seq, 3 * heads * head_dim]
    (SigLIP): out [n_views * seq, heads * head_dim]."""
    hid = heads * head_dim
    ld = qkv.stride(0)
    d = attention_desc(
        qkv, qkv[:, hid:], qkv[:, 2 * hid:], out, sq=seq, sk=seq, heads=1,
        head_dim=head_dim, n_problems=n_views * heads, zdiv=heads,
        q_tok_stride=ld, q_head_stride=0, q_zs=(seq * ld, head_dim),
        k_tok_stride=ld, k_zs=(seq * ld, head_dim),
        v_tok_stride=ld, v_zs=(seq * ld, head_dim),
        o_tok_stride=out.stride(0), o_head_stride=0,
        o_zs=(seq * out.stride(0), head_dim), scale=scale,
        kv_splits=kv_splits)
    run_attention(d)
    return out


# ---------------------------------------------------------------------------
# Data movement
# ---------------------------------------------------------------------------
def im2col_patches(images, patch, k_pad, out=None, scale=1.0, shift=0.0,
                   channels_last=False):
    """images [N, 3, H, W] (or [N, H, W, 3] with channels_last; bf16 or
    fp32) -> [N * (H/p) * (W/p), k_pad] bf16, columns (c, ky, kx)."""
    _check(images, 'images', dtype=None)
    if images.dtype not in (BF16, torch.float32):
        raise ValueError('images must be bf16 or fp32')
    if channels_last:
        n, h, w, c = images.shape
    else:
        n, c, h, w = images.shape
    if c != 3:
        raise ValueError('images must have 3 channels')
    rows = n * (h // patch) * (w // patch)
    if out is None:
        out = torch.empty(rows, k_pad, dtype=BF16, device=images.device)
    _check(out, 'out')
    _lib.call('fvx_im2col_patches', _ptr(images),
              int(images.dtype == torch.float32), int(bool(channels_last)),
              _ptr(out), n, h, w, patch, k_pad, float(scale), float(shift),
              _stream())
    return out


def embed_tokens(table, ids, out, scale=1.0, row_group=0, row_group_stride=0):
    _check(table, 'table')
    _check(ids, 'ids', dtype=torch.int64)
    _check(out, 'out', contiguous=False)
    _lib.call('fvx_embed_tokens', _ptr(table), _ptr(ids), _ptr(out),
              ids.numel(), table.shape[1], table.shape[0], float(scale),
              row_group, row_group_stride, _stream())
    return out


def copy_rows(src, dst, row_group=0, dst_group_stride=0):
    _check(src, 'src', contiguous=False)
    _check(dst, 'dst', contiguous=False)
    rows, sld = _rows_ld(src, 'src')
    _, dld = _rows_ld(dst, 'dst')
    _lib.call('fvx_copy_rows', _ptr(src), sld, _ptr(dst), dld, rows,
              src.shape[-1], row_group, dst_group_stride, _stream())
    return dst


def rope_table(max_pos, head_dim, theta=10000.0, device=None):
    """fp32 [max_pos, head_dim/2, 2] (cos, sin) of pos * inv_freq, with
    inv_freq = 1 / theta^(2i/head_dim) evaluated in fp32 as the HF Gemma
    rotary embedding does (condition_gemma.py:246-260)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64)
                           .float() / head_dim))
    pos = torch.arange(max_pos, dtype=torch.float32)
    ph = pos[:, None] * inv[None, :]
    t = torch.stack([torch.cos(ph), torch.sin(ph)], dim=-1).contiguous()
    return t.to(device) if device is not None else t


# ---------------------------------------------------------------------------
# Backward ops (guidance real-time chunking with use_vjp)
# ---------------------------------------------------------------------------
def _mapped_rows(t, name, rows, row_group, row_group_stride):
    """(leading dim) of a 2-D operand whose row m sits at
    (m / row_group) * row_group_stride + m % row_group; checks it covers
    the last mapped row."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f'{name} must be 2-D with unit column stride')
    if rows:
        last = rows - 1
        if row_group:
            last = (last // row_group) * row_group_stride + last % row_group
        if last >= t.shape[0]:
            raise ValueError(f'{name} has {t.shape[0]} rows, the map needs '
                             f'{last + 1}')
    return t.stride(0)


def rms_norm_backward(x, dy, *, out=None, out_bf16=None, out_frag=None,
                      dres=None, scale=None, gate=None, eps=1e-6, row_group=0,
                      row_group_stride=0):
    """dx of y = x r (1 + scale) (fvx_rms_norm_backward): dy fp32 [rows,
    cols] (compact); x bf16, dres / out fp32 and out_bf16 (= bf16(dx *
    gate)) 2-D views whose row m is (m / row_group) * row_group_stride +
    m % row_group; out_frag: a FragA receiving out_bf16's values.
    scale / gate: bf16 [cols] or None."""
    _check(dy, 'dy', dtype=torch.float32, contiguous=False)
    rows, ldy = _rows_ld(dy, 'dy')
    cols = dy.shape[-1]
    frag = _frag_out(out_frag, cols)
    if out is None and out_bf16 is None and frag is None:
        out = torch.empty(rows, cols, dtype=torch.float32, device=dy.device)
    _check(x, 'x', contiguous=False)
    ldx = _mapped_rows(x, 'x', rows, row_group, row_group_stride)
    args = []
    for t, nm, dt in ((dres, 'dres', torch.float32), (out, 'out', torch.float32),
                      (out_bf16, 'out_bf16', BF16)):
        if t is None:
            args.append(0)
            continue
        _check(t, nm, dtype=dt, contiguous=False)
        if t.shape[-1] != cols:
            raise ValueError(f'{nm} must have {cols} columns')
        args.append(_mapped_rows(t, nm, rows, row_group, row_group_stride))
    for t, nm in ((scale, 'scale'), (gate, 'gate')):
        _check(t, nm, contiguous=False, allow_none=True)
        if t is not None and (t.numel() < cols or t.stride(-1) != 1):
            raise ValueError(f'{nm} must hold {cols} contiguous values')
    if x.shape[-1] != cols:
        raise ValueError(f'x must have {cols} columns')
    _lib.call('fvx_rms_norm_backward', _ptr(x), ldx, _ptr(dy), ldy,
              _ptr(dres), args[0], _ptr(scale), _ptr(gate), _ptr(out),
              args[1], _ptr(out_bf16), args[2], frag, rows, cols, row_group,
              row_group_stride, float(eps), _stream())
    return out if out is not None else out_bf16


def _frag_out(f, width):
    """The buffer pointer of a FragA output of ``width`` columns, or None."""
    if f is None:
        return None
    if not isinstance(f, FragA) or f.k != width:
        raise ValueError(f'out_frag must be a FragA with k == {width}')
    _check(f.buf, 'out_frag')
    return f.buf.data_ptr()


def act_backward(act, inp, dy, out=None, out_frag=None):
    """GeGLU (act=ACT_BWD_GEGLU, inp = [gate | up] [rows, 2 cols]) or SiLU
    (inp = z [rows, cols]) backward; dy bf16 [rows, cols]; out bf16 like
    inp and / or out_frag, a FragA of the same width (fvx_act_backward)."""
    _check(inp, 'inp', contiguous=False)
    _check(dy, 'dy', contiguous=False)
    rows, ldy = _rows_ld(dy, 'dy')
    cols = dy.shape[-1]
    width = 2 * cols if act == _lib.ACT_BWD_GEGLU else cols
    if inp.shape[-1] != width:
        raise ValueError(f'inp must have {width} columns')
    frag = _frag_out(out_frag, width)
    if out is None and frag is None:
        out = torch.empty(rows, width, dtype=BF16, device=dy.device)
    ldo = 0
    if out is not None:
        _check(out, 'out', contiguous=False)
        _, ldo = _rows_ld(out, 'out')
    _, ldi = _rows_ld(inp, 'inp')
    _lib.call('fvx_act_backward', int(act), _ptr(inp), ldi, _ptr(dy), ldy,
              _ptr(out), ldo, frag, rows, cols, _stream())
    return out


def geglu_rows(gu, out=None, out_frag=None):
    """out = gelu_tanh(gu[:, :n]) * gu[:, n:] (bf16; fvx_geglu_rows), and /
    or the same into out_frag (a FragA with k == n)."""
    _check(gu, 'gu', contiguous=False)
    rows, ldgu = _rows_ld(gu, 'gu')
    n = gu.shape[-1] // 2
    frag = _frag_out(out_frag, n)
    if out is None and frag is None:
        out = torch.empty(rows, n, dtype=BF16, device=gu.device)
    ldo = 0
    if out is not None:
        _check(out, 'out', contiguous=False)
        _, ldo = _rows_ld(out, 'out')
    _lib.call('fvx_geglu_rows', _ptr(gu), ldgu, _ptr(out), ldo, frag, rows, n,
              _stream())
    return out


def attention_rows_backward(s, dp, ds, *, heads, n_keys, scale, kgrp=None,
                            qgrp=None, ds_t=None, p_t=None, key0=0,
                            n_suffix=0):
    """Masked softmax backward of one attention problem
    (fvx_attention_rows_backward): s, dp fp32 [rows, >= n_keys]; ds bf16
    [rows, n_cols]; ds_t / p_t bf16 [n_suffix, >= rows]."""
    _check(s, 's', dtype=torch.float32, contiguous=False)
    _check(dp, 'dp', dtype=torch.float32, contiguous=False)
    _check(ds, 'ds', contiguous=False)
    rows, lds = _rows_ld(s, 's')
    _, lddp = _rows_ld(dp, 'dp')
    _, ldds = _rows_ld(ds, 'ds')
    if dp.shape[0] != rows or ds.shape[0] != rows:
        raise ValueError('s, dp and ds must have the same rows')
    if rows % heads:
        raise ValueError('rows must be tokens * heads')
    for t, nm in ((kgrp, 'kgrp'), (qgrp, 'qgrp')):
        _check(t, nm, dtype=torch.int32, allow_none=True)
    if kgrp is not None and (kgrp.numel() < n_keys or qgrp is None
                             or qgrp.numel() < rows // heads):
        raise ValueError('kgrp must cover n_keys and qgrp every token')
    ldt = 0
    for t, nm in ((ds_t, 'ds_t'), (p_t, 'p_t')):
        if t is not None:
            _check(t, nm, contiguous=False)
            if t.shape[0] < n_suffix:
                raise ValueError(f'{nm} must have n_suffix rows')
            _, ld = _rows_ld(t, nm)
            if ldt and ld != ldt:
                raise ValueError('ds_t and p_t must share a leading dim')
            ldt = ld
    _lib.call('fvx_attention_rows_backward', _ptr(s), lds, _ptr(dp), lddp,
              _ptr(kgrp), _ptr(qgrp), _ptr(ds), ldds, _ptr(ds_t), _ptr(p_t),
              ldt, key0, n_suffix, rows, heads, n_keys, ds.shape[-1],
              float(scale), _stream())
    return ds


def attention_suffix_kv_backward(ds_t, p_t, q, dout, dk, dv):
    """dk = ds_t @ q, dv = p_t @ dout (fvx_attention_suffix_kv_backward):
    ds_t / p_t bf16 [n_suffix, >= rows], q / dout bf16 [rows, cols], dk / dv
    fp32 [n_suffix, cols]."""
    for t, nm in ((ds_t, 'ds_t'), (p_t, 'p_t'), (q, 'q'), (dout, 'dout')):
        _check(t, nm, contiguous=False)
    for t, nm in ((dk, 'dk'), (dv, 'dv')):
        _check(t, nm, dtype=torch.float32, contiguous=False)
    rows, ldq = _rows_ld(q, 'q')
    _, ldo = _rows_ld(dout, 'dout')
    ns, ldt = _rows_ld(ds_t, 'ds_t')
    if p_t.stride(0) != ldt or p_t.shape[0] != ns or dout.shape[0] != rows:
        raise ValueError('p_t must match ds_t and dout must match q')
    if dk.shape[0] < ns or dv.shape[0] < ns:
        raise ValueError('dk / dv need n_suffix rows')
    _lib.call('fvx_attention_suffix_kv_backward', _ptr(ds_t), _ptr(p_t), ldt,
              _ptr(q), ldq, _ptr(dout), ldo, _ptr(dk), dk.stride(0), _ptr(dv),
              dv.stride(0), ns, rows, q.shape[-1], _stream())
    return dk, dv


def transpose(src, dst):
    """dst[..., c, r] = src[..., r, c] for bf16 [rows, cols] or [batch, rows,
    cols] views (unit column stride)."""
    _check(src, 'src', contiguous=False)
    _check(dst, 'dst', contiguous=False)
    s3 = src if src.dim() == 3 else src[None]
    d3 = dst if dst.dim() == 3 else dst[None]
    if (s3.dim() != 3 or d3.dim() != 3 or s3.stride(-1) != 1 or d3.stride(-1) != 1
            or d3.shape != (s3.shape[0], s3.shape[2], s3.shape[1])):
        raise ValueError('transpose: dst must be src with its last two dims '
                         'swapped, both with unit column stride')
    _lib.call('fvx_transpose_bf16', _ptr(src), s3.stride(1), s3.stride(0),
              _ptr(dst), d3.stride(1), d3.stride(0), s3.shape[1], s3.shape[2],
              s3.shape[0], _stream())
    return dst


def rope_backward(dq, dk, dv, rope, positions, out, n_q_heads, head_dim,
                  out_frag=None):
    """out bf16 [rows, (n_q_heads + 2) * head_dim] = [dq, dk rotated back |
    dv] (fvx_rope_backward); dk / dv fp32 2-D views, dq one too or a 3-D
    [parts, rows, cols] stack of partials (summed)."""
    for t, nm in ((dq, 'dq'), (dk, 'dk'), (dv, 'dv'), (rope, 'rope')):
        _check(t, nm, dtype=torch.float32, contiguous=(nm == 'rope'))
    _check(positions, 'positions', dtype=torch.int32)
    frag = _frag_out(out_frag, (n_q_heads + 2) * head_dim)
    if out is not None:
        _check(out, 'out', contiguous=False)
    parts, pstride = 1, 0
    if dq.dim() == 3:
        parts, pstride = dq.shape[0], dq.stride(0)
        dq = dq[0]
    rows, ldq = _rows_ld(dq, 'dq')
    if positions.numel() < rows or dk.shape[0] != rows or dv.shape[0] != rows:
        raise ValueError('dq, dk, dv and positions must cover the same rows')
    _lib.call('fvx_rope_backward', _ptr(dq), ldq, parts, pstride, _ptr(dk),
              dk.stride(0), _ptr(dv), dv.stride(0), _ptr(rope), _ptr(positions),
              _ptr(out), out.stride(0) if out is not None else 0, frag, rows,
              n_q_heads, head_dim, _stream())
    return out


def attention_backward_parts(n_keys):
    """Key-tile partials of fvx_attention_backward's dq."""
    return int(_lib.load().fvx_attention_backward_parts(n_keys))


def attention_backward(q, o, dout, k, v, kt, dq, stats, *, heads, scale,
                       kgrp=None, qgrp=None, ds_t=None, p_t=None, key0=0,
                       n_suffix=0, vt=None, refresh=(0, 0)):
    """Fused decode-shape attention backward (fvx_attention_backward) for
    n problems: q / o / dout bf16 [n, rows, 256]; k / v bf16 [n, >= n_keys,
    256] rows with n_keys = k.shape[1]; kt bf16 [n, 256, kt_ld] (zero past
    n_keys); dq fp32 [parts, n * rows, 256]; stats fp32 scratch of
    2 * n * parts * rows; kgrp int32 [n, >= n_keys], qgrp [n, rows / heads];
    ds_t / p_t bf16 [n, n_suffix, >= rows]; vt bf16 [n, 256, >= n_keys] (the
    value cache) with ``refresh`` = (first key, count): those keys' kt
    columns and v rows are first rewritten from k and vt."""
    d = _lib.AttnBwdDesc()
    n, rows, hd = q.shape
    nk = k.shape[1]
    for t, nm in ((q, 'q'), (o, 'o'), (dout, 'dout')):
        _check(t, nm, contiguous=False)
        if t.shape != q.shape or t.stride(1) != hd or t.stride(2) != 1:
            raise ValueError(f'{nm} must be [n, rows, head_dim] with packed rows')
    for t, nm in ((k, 'k'), (v, 'v')):
        _check(t, nm, contiguous=False)
        if t.shape[0] != n or t.shape[2] != hd or t.stride(1) != hd or t.stride(2) != 1:
            raise ValueError(f'{nm} must be [n, keys, head_dim] with packed rows')
    _check(kt, 'kt', contiguous=False)
    if kt.shape[:2] != (n, hd) or kt.stride(2) != 1 or kt.stride(1) < nk:
        raise ValueError('kt must be [n, head_dim, >= n_keys]')
    parts = attention_backward_parts(nk)
    _check(dq, 'dq', dtype=torch.float32)
    if dq.shape != (parts, n * rows, hd):
        raise ValueError(f'dq must be [{parts}, {n * rows}, {hd}]')
    _check(stats, 'stats', dtype=torch.float32)
    if stats.numel() < 2 * n * parts * rows:
        raise ValueError('stats is too small')
    d.q, d.q_zs = q.data_ptr(), q.stride(0)
    d.o, d.o_zs = o.data_ptr(), o.stride(0)
    d.dout, d.do_zs = dout.data_ptr(), dout.stride(0)
    d.k, d.k_zs = k.data_ptr(), k.stride(0)
    d.v, d.v_zs = v.data_ptr(), v.stride(0)
    d.kt, d.kt_ld, d.kt_zs = kt.data_ptr(), kt.stride(1), kt.stride(0)
    if vt is not None:
        _check(vt, 'vt', contiguous=False)
        if vt.shape[:2] != (n, hd) or vt.stride(2) != 1 or vt.shape[2] < nk:
            raise ValueError('vt must be [n, head_dim, >= n_keys]')
        d.vt, d.vt_ld, d.vt_zs = vt.data_ptr(), vt.stride(1), vt.stride(0)
        d.refresh_key0, d.refresh_n = refresh
    if kgrp is not None:
        _check(kgrp, 'kgrp', dtype=torch.int32, contiguous=False)
        _check(qgrp, 'qgrp', dtype=torch.int32, contiguous=False)
        if (kgrp.shape[-1] < nk or qgrp.shape[-1] < rows // heads
                or kgrp.stride(-1) != 1 or qgrp.stride(-1) != 1):
            raise ValueError('kgrp must cover the keys and qgrp every token')
        d.kgrp, d.kgrp_zs = kgrp.data_ptr(), kgrp.stride(0) if kgrp.dim() > 1 else 0
        d.qgrp, d.qgrp_zs = qgrp.data_ptr(), qgrp.stride(0) if qgrp.dim() > 1 else 0
    d.stats = stats.data_ptr()
    d.dq, d.dq_parts = dq.data_ptr(), parts
    if ds_t is not None or p_t is not None:
        for t, nm in ((ds_t, 'ds_t'), (p_t, 'p_t')):
            _check(t, nm)
            if t.shape[:2] != (n, n_suffix) or t.shape[2] < rows:
                raise ValueError(f'{nm} must be [n, n_suffix, >= rows]')
        d.ds_t, d.p_t = _ptr(ds_t), _ptr(p_t)
        d.ldt, d.t_zs = ds_t.stride(1), ds_t.stride(0)
    d.rows, d.heads, d.head_dim = rows, heads, hd
    d.n_keys, d.key0, d.n_suffix, d.n_problems = nk, key0, n_suffix, n
    d.scale = float(scale)
    _lib.call('fvx_attention_backward', ctypes.byref(d), _stream())
    return dq


def rtc_vjp_error(x, u, prev, w, e, omt):
    """e = bf16(w[m % period] (prev - x + omt u)) (fvx_rtc_vjp_error); x, u,
    prev fp32 [rows, cols]; w fp32 [period]."""
    for t, nm in ((x, 'x'), (u, 'u'), (prev, 'prev'), (w, 'w')):
        _check(t, nm, dtype=torch.float32, contiguous=False)
    _check(e, 'e', contiguous=False)
    rows, cols = x.shape
    _lib.call('fvx_rtc_vjp_error', _ptr(x), x.stride(0), _ptr(u), u.stride(0),
              _ptr(prev), prev.stride(0), _ptr(w), _ptr(e), e.stride(0), rows,
              cols, w.numel(), float(omt), _stream())
    return e


def rtc_vjp_update(x, u, prev, w, g, gw, omt, dt, x_bf16=None):
    """x <- x + dt u - dt gw e + dt gw omt g, e = w (prev - x + omt u)
    (fvx_rtc_vjp_update); gw: device fp32 scalar (a 1-element view)."""
    for t, nm in ((x, 'x'), (u, 'u'), (prev, 'prev'), (w, 'w'), (g, 'g'),
                  (gw, 'gw')):
        _check(t, nm, dtype=torch.float32, contiguous=False)
    _check(x_bf16, 'x_bf16', contiguous=False, allow_none=True)
    rows, cols = x.shape
    _lib.call('fvx_rtc_vjp_update', _ptr(x), x.stride(0), _ptr(x_bf16),
              x_bf16.stride(0) if x_bf16 is not None else 0, _ptr(u),
              u.stride(0), _ptr(prev), prev.stride(0), _ptr(w), _ptr(g),
              g.stride(0), _ptr(gw), rows, cols, w.numel(), float(omt),
              float(dt), _stream())
    return x



# ---------------------------------------------------------------------------
# Camera-frame preprocessing
# ---------------------------------------------------------------------------
def resize_normalize(src, out, *, hwc, region=None, pad_value=0.0,
                     filter=_lib.RESIZE_LINEAR, round_u8=False, swap_rb=False,
                     mean=(0.0, 0.0, 0.0), den=(1.0, 1.0, 1.0), pre_div=1.0):
    """n RGB images -> fp32 CHW planes ``out`` [n, 3, H, W] (a view with unit
    plane strides; the image stride may be larger, e.g. one view of the
    model's [B, 3 * views, H, W] buffer).  ``src``: uint8 or fp32 [n, h, w, 3]
    (``hwc``) or [n, 3, h, w], contiguous per image.  ``region`` = (off_y,
    off_x, rh, rw): where the resized picture goes, pad_value elsewhere
    (default: the whole output; a 3-sequence pads each channel with its own
    value).  out = (v / pre_div - mean[c]) / den[c]."""
    if src.dtype not in (torch.uint8, torch.float32):
        raise ValueError(f'src must be uint8 or fp32, got {src.dtype}')
    if src.dim() != 4 or (src.shape[3] if hwc else src.shape[1]) != 3:
        raise ValueError(f'src must be [n, h, w, 3] (hwc) or [n, 3, h, w], '
                         f'got {tuple(src.shape)}')
    _check(out, 'out', dtype=torch.float32, contiguous=False)
    n = src.shape[0]
    h, w = (src.shape[1], src.shape[2]) if hwc else (src.shape[2], src.shape[3])
    if src.stride()[1:] != torch.empty(src.shape[1:]).stride():
        raise ValueError('src images must be contiguous')
    if (out.dim() != 4 or out.shape[0] != n or out.shape[1] != 3 or
            out.stride(3) != 1 or out.stride(2) != out.shape[3] or
            out.stride(1) != out.shape[2] * out.shape[3]):
        raise ValueError('out must be [n, 3, H, W] with contiguous planes')
    H, W = out.shape[2], out.shape[3]
    off_y, off_x, rh, rw = region if region is not None else (0, 0, H, W)
    d = _lib.ImageDesc()
    d.src, d.src_u8, d.src_hwc = src.data_ptr(), int(src.dtype == torch.uint8), int(hwc)
    d.n, d.src_h, d.src_w = n, h, w
    d.src_img_stride = src.stride(0) if n > 1 else 3 * h * w
    d.dst, d.dst_h, d.dst_w = out.data_ptr(), H, W
    d.dst_img_stride = out.stride(0) if n > 1 else 3 * H * W
    d.rh, d.rw, d.off_y, d.off_x = rh, rw, off_y, off_x
    if isinstance(pad_value, (tuple, list)):
        if len(pad_value) != 3:
            raise ValueError('a per-channel pad_value needs 3 values')
        d.pad_per_channel = 1
        for c in range(3):
            d.pad_rgb[c] = float(pad_value[c])
    else:
        d.pad_value = float(pad_value)
    d.filter = int(filter)
    d.round_u8, d.swap_rb, d.pre_div = int(round_u8), int(swap_rb), float(pre_div)
    for c in range(3):
        d.mean[c], d.den[c] = float(mean[c]), float(den[c])
    _lib.call('fvx_resize_normalize', ctypes.byref(d), _stream())
    return out
