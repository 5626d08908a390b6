"""Guidance real-time chunking with ``use_vjp``: the action expert's
vector-Jacobian product on the GPU.

apply_rtc_guidance (fluxvla/engines/utils/rtc_guidance.py:107-155, under
_predict_action_guidance_rtc, pi0_flowmatching.py:671-700) takes, with
use_vjp, the correction c = (d x_1 / d x_t)^T e from torch autograd through
the whole denoiser, x_1 = x_t - (1 - t) u(x_t) for the model velocity u and
e = w (prev - x_1) on the previous chunk's rows.  Here one Euler step is

  forward   the expert as in the plain loop, keeping each layer's input
            stream X[i], its post-attention stream X2[i], its rotated
            queries Q[i] (the key/value cache already holds the suffix
            keys and values), its attention output and its MLP's [gate |
            up] rows GU[i] (written by the GeGLU GEMM beside its product);
            u from a PLAIN fp32 GEMM of action_out_proj;
  error     e = bf16(w (prev - x + (1 - t) u))                (one kernel);
  backward  g = J_u^T e layer by layer, last to first:
              down:       dh = (gate2 dX3) @ W_down
              GeGLU:      the activation backward on GU[i],
                          da = d[gate | up] @ [Wg; Wu]
              norm:       dX2 = dX3 + RMSNorm-backward(X2, da)
              O:          dO = (gate1 dX2) @ W_o
              attention:  one fused MFMA backward (S = Q K^T, P from the
                          rows' log-sum-exp, dP = dO V^T, dS, dQ = dS K in
                          key-tile partials), then dK = dS^T Q and dV = P^T
                          dO on the suffix keys (the prefix cache is a
                          constant of x_t), RoPE backward summing dQ
              QKV:        da = d[q | k | v] @ W_qkv
              norm:       dX = dX2 + RMSNorm-backward(X, da)
            and through the suffix embedding (PI0: action-time MLP with
            its SiLU; PI0.5: action_in_proj) to g = dL/dx_t;
  update    x <- x + dt u - dt gw e + dt gw (1 - t) g              (one kernel).

The weights' products run through fvx_gemm on [in, out] copies of the
prepared [out, in] weights (fp8 weights dequantized to bf16; fragment-major
for the M <= 64 GEMMs of bs=1); the attention backward reads the key cache,
a transposed copy of it and a row-major copy of the value cache.  All of it is part of the captured chunk
graph: per-request values (previous chunk, weights, guidance weights) are
device buffers.
"""
import torch

from . import _lib
from . import kernels as K

BF16 = torch.bfloat16


def _weight_t(w):
    """bf16 [in, out] copy of a prepared [out, in] weight (bf16 or row-major
    fp8, dequantized): the B operand of dX = dY @ W."""
    if isinstance(w, K.Fp8Weight):
        w = w.dequantize()
    return w.t().contiguous().to(BF16)


class ExpertVJP:
    """Transposed weights, saved activations and scratch of the VJP step
    for one model; buffers per batch size."""

    def __init__(self, model):
        self.m = m = model
        cfg = m.cfg
        self.wT = []
        for L in m.exp['layers']:
            gu = torch.cat([_weight_t(L['gate_w']), _weight_t(L['up_w'])], 1)
            self.wT.append({'qkv': _weight_t(L['qkv_w']),
                            'o': _weight_t(L['o_w']),
                            'gu': gu.contiguous(),
                            'down': _weight_t(L['down_w'])})
        self.out_t = _weight_t(m.act_out['w'])       # [hid, action_dim]
        if cfg.pi05:
            self.in_t = _weight_t(m.act_in['w'])     # [action_dim, hid]
        else:
            self.mo_t = _weight_t(m.mlp_out['w'])    # [proj_width, hid]
            self.mi_t = _weight_t(m.mlp_in_x)        # [action_dim, proj]
        # fragment-major copies for the M <= 64 GEMMs (bs = 1)
        F = K.FragB.pack
        self.wT_f = [{nm: F(w) for nm, w in L.items()} for L in self.wT]
        self.out_t_f = F(self.out_t)
        if cfg.pi05:
            self.in_t_f = F(self.in_t)
        else:
            self.mo_t_f, self.mi_t_f = F(self.mo_t), F(self.mi_t)
        self.scale = cfg.head_dim ** -0.5
        self._bufs = {}

    def _frag(self, B):
        """The expert's GEMMs have M = B * suffix_len rows: fragment-major
        weights when that is <= 64."""
        return B * self.m.cfg.suffix_len <= 64

    # -- buffers -------------------------------------------------------------
    def buffers(self, B):
        if B in self._bufs:
            return self._bufs[B]
        m, cfg, dev = self.m, self.m.cfg, self.m.device
        S, Ss, D, H = cfg.prefix_len, cfg.suffix_len, cfg.head_dim, cfg.heads
        na, hid, mlp = cfg.n_action_steps, cfg.exp_hidden, cfg.exp_mlp
        T, nL, ad = m.kv_len, cfg.exp_layers, cfg.max_action_dim
        R = Ss * H
        parts = K.attention_backward_parts(S + Ss)

        def e(*shape, dt=BF16):
            return torch.empty(*shape, dtype=dt, device=dev)

        def z(*shape, dt=BF16):
            return torch.zeros(*shape, dtype=dt, device=dev)
        v = {
            'X': e(nL + 1, B * Ss, hid), 'X2': e(nL, B * Ss, hid),
            'Q': e(nL, B * Ss, H * D), 'CTX': e(nL, B * Ss, H * D),
            'h': e(B * Ss, mlp), 'xn': e(B * Ss, hid), 'gate': e(B * Ss, hid),
            # key cache transposed [layer][batch][dim][token] and value cache
            # row-major [layer][batch][token][dim]; the columns / rows past
            # the keys stay zero (the dQ GEMM's K runs over them)
            'kT': z(nL, B, D, T), 'vr': z(nL, B, T, D),
            'u': e(B * na, ad, dt=torch.float32), 'e': e(B * na, ad),
            'g': e(B * na, ad, dt=torch.float32),
            'dx': [e(B * Ss, hid, dt=torch.float32) for _ in range(2)],
            'da': e(B * Ss, hid, dt=torch.float32), 'a': e(B * Ss, hid),
            'dh': e(B * Ss, mlp), 'GU': e(nL, B * Ss, 2 * mlp),
            'dgu': e(B * Ss, 2 * mlp), 'dctx': e(B, Ss, H * D),
            'ds_t': e(B, Ss, R), 'p_t': e(B, Ss, R),
            'dq': e(parts, B * R, D, dt=torch.float32),
            'stats': e(2 * B * parts * R, dt=torch.float32),
            'dk': e(B * Ss, D, dt=torch.float32),
            'dv': e(B * Ss, D, dt=torch.float32),
            'dqkv': e(B * Ss, (H + 2) * D),
        }
        if self._frag(B):
            # fragment-major copies of the M <= 64 GEMMs' A operands
            F = lambda k: K.FragA.empty(k, dev).rows(B * Ss)  # noqa: E731
            v['f'] = {'x': F(hid), 'x2': F(hid), 'ctx': F(H * D), 'h': F(mlp),
                      'a': F(hid), 'dgu': F(2 * mlp), 'dqkv': F((H + 2) * D)}
        if not cfg.pi05:
            v['z'] = e(B * na, cfg.proj_width)
            v['dsh'] = e(B * na, cfg.proj_width)
            v['dz'] = e(B * na, cfg.proj_width)
        self._bufs[B] = v
        return v

    # -- the chunk -------------------------------------------------------------
    def decoder(self, b, B):
        """The Euler loop with the VJP-corrected guidance update (replaces
        PI0Inference.transformer_decoder for this method)."""
        m, cfg = self.m, self.m.cfg
        v = self.buffers(B)
        S, Ss, hid = cfg.prefix_len, cfg.suffix_len, cfg.exp_hidden
        nL = cfg.exp_layers
        # the prefix part of every layer's transposed key / row-major value
        # cache, once per chunk
        kc = b['kc'].view(nL * B, m.kv_len, cfg.head_dim)
        vc = b['vc'].view(nL * B, cfg.head_dim, m.kv_len)
        K.transpose(kc[:, :S], v['kT'].view(nL * B, cfg.head_dim, m.kv_len)[:, :, :S])
        K.transpose(vc[:, :, :S], v['vr'].view(nL * B, m.kv_len, cfg.head_dim)[:, :S])
        if not cfg.pi05:
            K.gemm(b['states'], m.state['w'], out=b['suf_res'],
                   bias=m.state['b'], row_group=1, row_group_stride=Ss)
        for step in range(len(m.times)):
            self.forward(b, B, step)
            self.backward(b, B, step)

    def forward(self, b, B, step):
        """Suffix embedding, expert layers with saved streams, u and e."""
        m, cfg, v = self.m, self.m.cfg, self._bufs[B]
        S, Ss, D, H = cfg.prefix_len, cfg.suffix_len, cfg.head_dim, cfg.heads
        na, hid, T = cfg.n_action_steps, cfg.exp_hidden, m.kv_len
        X, X2, Q = v['X'], v['X2'], v['Q']
        xt_b = b['xt_bf16'].view(B * na, -1)
        fr = self._frag(B)
        f = v.get('f') if fr else None
        fc = (lambda nm: f[nm] if f else None)  # noqa: E731
        if cfg.pi05:
            K.gemm(xt_b, m.act_in_f if fr else m.act_in['w'], out=X[0],
                   bias=m.act_in['b'])
        else:
            h = b['suf_h']  # the state rows stay zero
            w_mi = m.mlp_in_x_f if fr else m.mlp_in_x
            K.gemm(xt_b, w_mi, out=h[1:], bias_f32=m.step_bias[step],
                   act=_lib.ACT_SILU, row_group=na, row_group_stride=Ss)
            K.gemm(xt_b, w_mi, out=v['z'], bias_f32=m.step_bias[step])
            K.gemm(h, m.mlp_out_f if fr else m.mlp_out['w'], out=X[0],
                   residual=b['suf_res'], c_frag=fc('x'))
        st = m.styles[step] if cfg.pi05 else None
        layers = m.exp_f if fr else m.exp['layers']
        for i, L in enumerate(layers):
            kc, vc = b['kc'][i], b['vc'][i]
            x = X[i]
            if cfg.pi05:
                K.adarms_norm(x, st[2 * i:2 * i + 1], out=v['xn'],
                              gate_out=v['gate'], eps=cfg.rms_eps)
                a, rn = v['xn'], None
            else:
                a, rn = (f['x'] if f else x), cfg.rms_eps
            # the suffix keys / values also into the attention backward's
            # transposed-key and row-major value copies
            K.gemm_qkv_rope(a, L['qkv_w'], m.rope, b['pos_suf'], Q[i],
                            kc.view(B * T, D)[S:], vc[:, :, S:], H, D,
                            rownorm_eps=rn, row_group=Ss, row_group_stride=T,
                            v_ld=T, k_t_out=v['kT'][i][:, :, S:], kt_ld=T,
                            v_rows_out=v['vr'][i].view(B * T, D)[S:])
            ctx = v['CTX'][i]
            K.mqa_attention(Q[i].view(B, Ss, H * D), kc[:, :S + Ss], vc,
                            ctx.view(B, Ss, H * D), kgrp=b['kgrp'],
                            qgrp=b['qgrp_suf'], v_transposed=True,
                            o_frag=fc('ctx'))
            gate = v['gate'] if cfg.pi05 else None
            K.gemm(f['ctx'] if f else ctx, L['o_w'], out=X2[i], residual=x,
                   gate=gate, c_frag=None if cfg.pi05 else fc('x2'))
            # the GeGLU GEMM, keeping its [gate | up] values for the backward
            if cfg.pi05:
                K.adarms_norm(X2[i], st[2 * i + 1:2 * i + 2], out=v['xn'],
                              gate_out=v['gate'], eps=cfg.rms_eps)
                a2, rn = v['xn'], None
            else:
                a2, rn = (f['x2'] if f else X2[i]), cfg.rms_eps
            K.gemm_geglu(a2, L['gate_w'], L['up_w'], out=v['h'],
                         rownorm_eps=rn, c_frag=fc('h'), gu_out=v['GU'][i])
            K.gemm(f['h'] if f else v['h'], L['down_w'], out=X[i + 1],
                   residual=X2[i], gate=gate,
                   c_frag=None if cfg.pi05 else fc('x'))
        lead = Ss - na
        last = X[-1].view(B, Ss, hid)
        w_out = m.act_out_f if fr else m.act_out['w']
        if cfg.pi05:
            K.adarms_norm(X[-1], st[-1:], out=v['xn'], eps=cfg.rms_eps)
            K.gemm(v['xn'], w_out, out=v['u'], bias=m.act_out['b'],
                   out_f32=True)
        else:
            K.gemm(last[:, lead:], w_out, out=v['u'], bias=m.act_out['b'],
                   rownorm_eps=cfg.rms_eps, out_f32=True)
        K.rtc_vjp_error(b['xt'].view(B * na, -1), v['u'],
                        b['rtc_prev'].view(B * na, -1), b['rtc_w'], v['e'],
                        m._rtc_omt[step])

    def backward(self, b, B, step):
        """g = J_u^T e through the expert and the suffix embedding, then the
        corrected Euler update."""
        m, cfg, v = self.m, self.m.cfg, self._bufs[B]
        S, Ss, D, H = cfg.prefix_len, cfg.suffix_len, cfg.head_dim, cfg.heads
        na, hid, mlp, T = (cfg.n_action_steps, cfg.exp_hidden, cfg.exp_mlp,
                           m.kv_len)
        nk, R, eps = S + Ss, Ss * H, cfg.rms_eps
        X, X2, Q = v['X'], v['X2'], v['Q']
        lead = Ss - na
        w = hid
        st = m.styles[step] if cfg.pi05 else None

        def gate2(i):  # the MLP branch's gate of layer i (PI0.5)
            return st[2 * i + 1, 2 * w:] if (cfg.pi05 and i >= 0) else None

        nL = len(m.exp['layers'])
        fr = self._frag(B)
        wts = self.wT_f if fr else self.wT
        f = v.get('f') if fr else None
        af = f['a'] if f else None
        a_in = af if f else v['a']  # the A operand of the backward GEMMs
        dx, dx2 = v['dx']
        # d(final norm output) = e @ W_out, then the final norm's backward
        # onto the action rows (the state row of PI0 gets none)
        dxn = v['da'][:B * na]
        K.gemm(v['e'], self.out_t_f if fr else self.out_t, out=dxn,
               out_f32=True)
        if cfg.pi05:
            K.rms_norm_backward(X[-1], dxn, out=dx, out_bf16=v['a'],
                                out_frag=af, scale=st[-1, :w],
                                gate=gate2(nL - 1), eps=eps)
        else:
            dx.zero_()
            v['a'].zero_()
            K.rms_norm_backward(X[-1][lead:], dxn, out=dx[lead:],
                                out_bf16=v['a'][lead:], eps=eps,
                                row_group=na, row_group_stride=Ss)
            if af is not None:  # all rows, the zero state rows included
                K.pack_frag(v['a'], af)
        for i in range(nL - 1, -1, -1):
            wt = wts[i]
            # MLP: dh = (gate2 dX3) @ W_down, then GeGLU's backward on the
            # [gate | up] rows the forward kept
            K.gemm(a_in, wt['down'], out=v['dh'])
            if f:
                K.act_backward(_lib.ACT_BWD_GEGLU, v['GU'][i], v['dh'],
                               out_frag=f['dgu'])
            else:
                K.act_backward(_lib.ACT_BWD_GEGLU, v['GU'][i], v['dh'],
                               out=v['dgu'])
            K.gemm(f['dgu'] if f else v['dgu'], wt['gu'], out=v['da'],
                   out_f32=True)
            K.rms_norm_backward(
                X2[i], v['da'], dres=dx, out=dx2,
                out_bf16=None if f else v['a'], out_frag=af,
                scale=st[2 * i + 1, :w] if cfg.pi05 else None,
                gate=st[2 * i, 2 * w:] if cfg.pi05 else None, eps=eps)
            # attention: dO = (gate1 dX2) @ W_o
            K.gemm(a_in, wt['o'], out=v['dctx'].view(B * Ss, -1))
            self._attention_backward(b, B, i)
            K.gemm(f['dqkv'] if f else v['dqkv'], wt['qkv'], out=v['da'],
                   out_f32=True)
            # the last one (layer 0) also row-major: the suffix embedding's
            # backward reads the action rows
            K.rms_norm_backward(
                X[i], v['da'], dres=dx2, out=dx,
                out_bf16=v['a'] if (i == 0 or not f) else None, out_frag=af,
                scale=st[2 * i, :w] if cfg.pi05 else None, gate=gate2(i - 1),
                eps=eps)
        # suffix embedding: g = dL/dx_t
        if cfg.pi05:
            K.gemm(a_in, self.in_t_f if fr else self.in_t, out=v['g'],
                   out_f32=True)
        else:
            a = v['a'].view(B, Ss, hid)[:, lead:]
            K.gemm(a, self.mo_t_f if fr else self.mo_t, out=v['dsh'])
            K.act_backward(_lib.ACT_BWD_SILU, v['z'], v['dsh'], out=v['dz'])
            K.gemm(v['dz'], self.mi_t_f if fr else self.mi_t, out=v['g'],
                   out_f32=True)
        K.rtc_vjp_update(b['xt'].view(B * na, -1), v['u'],
                         b['rtc_prev'].view(B * na, -1), b['rtc_w'], v['g'],
                         b['rtc_gw'][step:step + 1], m._rtc_omt[step], m.dt,
                         x_bf16=b['xt_bf16'].view(B * na, -1))

    def _attention_backward(self, b, B, i):
        """dq, dk, dv of layer i's attention from dO (v['dctx']), packed with
        the RoPE backward into v['dqkv']: the fused attention backward over
        the batch's problems, then the suffix keys' dK / dV per sample."""
        m, cfg, v = self.m, self.m.cfg, self._bufs[B]
        S, Ss, D, H = cfg.prefix_len, cfg.suffix_len, cfg.head_dim, cfg.heads
        nk, R = S + Ss, Ss * H
        kc, vc = b['kc'][i], b['vc'][i]
        kT, vr = v['kT'][i], v['vr'][i]
        q3 = v['Q'][i].view(B, R, D)
        do3 = v['dctx'].view(B, R, D)
        K.attention_backward(q3, v['CTX'][i].view(B, R, D), do3, kc[:, :nk],
                             vr[:, :nk], kT, v['dq'], v['stats'], heads=H,
                             scale=self.scale, kgrp=b['kgrp'],
                             qgrp=b['qgrp_suf'], ds_t=v['ds_t'], p_t=v['p_t'],
                             key0=S, n_suffix=Ss)
        for z in range(B):
            rows = slice(z * Ss, (z + 1) * Ss)
            K.attention_suffix_kv_backward(v['ds_t'][z], v['p_t'][z], q3[z],
                                           do3[z], v['dk'][rows], v['dv'][rows])
        f = v.get('f') if self._frag(B) else None
        K.rope_backward(v['dq'].view(-1, B * Ss, H * D), v['dk'], v['dv'],
                        m.rope, b['pos_suf'], None if f else v['dqkv'], H, D,
                        out_frag=f['dqkv'] if f else None)
