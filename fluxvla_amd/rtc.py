"""Real-time chunking (RTC) of the Euler loop: host-side tables.

The reference runs RTC in its eager loop (PI0FlowMatching.predict_action,
fluxvla/models/vlas/pi0_flowmatching.py:651-700, 744-785) with the guidance
helpers of fluxvla/engines/utils/rtc_guidance.py.  Here both methods run
inside the captured chunk graph, folded into kernels that already run:

* prefix: the first ``prefix_len`` positions of the chunk are the previous
  chunk's actions before every denoise call and at the end, and they are
  denoised at time 0.  The Euler GEMM stores the previous actions on those
  rows, the suffix-embedding GEMM (PI0) adds the time-0 bias on them and the
  adaRMS norms (PI0.5) use the time-0 style row; the prefix length is a
  device int32, so one graph serves every length.
* guidance (without VJP): v <- v + gw * w_r * (prev - x_1) in the reference's
  0 = noise time convention, x_1 = x_t - time * v.  Folded into the Euler
  update as x + dt v + cw_r (prev - x + time v) with cw_r = -dt * gw(step) *
  w_r, read from a per-step table that depends only on the request's RTC
  settings.
* guidance with use_vjp ('guidance_vjp'): the error pulled back through the
  expert's Jacobian, J^T e, by the backward pass of fluxvla_amd.vjp; the
  update reads the prefix weights and per-step guidance weights from device
  tables (guidance_vjp_tables).

``compute_prefix_weights`` and ``compute_guidance_weight`` keep the
reference's names and arguments (rtc_guidance.py:28-104).
"""
import math

import torch

METHODS = ('prefix', 'guidance')


def compute_prefix_weights(n_action_steps, prefix_len, decay_end,
                           schedule='exp', device='cpu'):
    """Per-position guidance weights (rtc_guidance.py:28-80): 1 on the
    locked prefix, then from prefix_len to decay_end a decay over
    f = i / max(decay_len - 1, 1): 'exp' exp(-3 f), 'linear' 1 - f, 'ones'
    1, 'zeros' 0; 0 elsewhere.  fp32 [n_action_steps]."""
    w = [0.0] * n_action_steps
    if prefix_len > 0:
        for i in range(min(prefix_len, n_action_steps)):
            w[i] = 1.0
        decay_len = decay_end - prefix_len
        for i in range(max(decay_len, 0)):
            pos = prefix_len + i
            if pos >= n_action_steps:
                break
            f = i / max(decay_len - 1, 1)
            if schedule == 'exp':
                w[pos] = math.exp(-3.0 * f)
            elif schedule == 'linear':
                w[pos] = 1.0 - f
            elif schedule == 'ones':
                w[pos] = 1.0
            elif schedule == 'zeros':
                w[pos] = 0.0
            else:
                raise ValueError(f'Unknown schedule: {schedule}')
    return torch.tensor(w, dtype=torch.float32, device=device)


def compute_guidance_weight(t, max_guidance_weight):
    """Guidance weight of one step (rtc_guidance.py:83-104); t is the
    denoising progress, 0 = noise, 1 = clean.  Strong early, weak late:
    min((1 - t) / t * (t^2 + (1 - t)^2) / (1 - t)^2, max), t and 1 - t
    clamped to 1e-6."""
    tc = max(t, 1e-6)
    omt = max(1.0 - t, 1e-6)
    return min(omt / tc * (tc * tc + omt * omt) / (omt * omt),
               max_guidance_weight)


def select_method(prev_actions, prefix_len, rtc_config):
    """The loop predict_action runs (pi0_flowmatching.py:753-756): the
    configured method (default 'prefix') when prev_actions, prefix_len > 0
    and rtc_config are all given, else None (the plain loop)."""
    if prev_actions is None or prefix_len <= 0 or not rtc_config:
        return None
    method = rtc_config.get('method', 'prefix')
    if method not in METHODS:
        # the reference falls through to the plain loop for other names
        return None
    if method == 'guidance' and rtc_config.get('use_vjp', False):
        # the correction pulled back through the expert's Jacobian
        # (fluxvla_amd.vjp)
        return 'guidance_vjp'
    return method


def pad_prev_actions(prev_actions, max_action_dim, ori_action_dim):
    """prev_actions zero-padded to max_action_dim when the model has an
    ori_action_dim (pi0_flowmatching.py:747-751)."""
    d = prev_actions.shape[-1]
    if ori_action_dim is not None and d < max_action_dim:
        prev_actions = torch.nn.functional.pad(prev_actions,
                                               (0, max_action_dim - d))
    if prev_actions.shape[-1] != max_action_dim:
        raise ValueError(f'prev_actions has {prev_actions.shape[-1]} action '
                         f'dims, the chunk has {max_action_dim}')
    return prev_actions


def guidance_omt(times):
    """The (1 - t) factor of each step's predicted clean chunk x_1 = x_t +
    v_rtc (1 - t), t = 1 - time (rtc_guidance.py:138-140 with
    pi0_flowmatching.py:691-697); a constant of the captured graph."""
    return [max(1.0 - (1.0 - time), 1e-6) for time in times]


def guidance_cw(times, dt, n_action_steps, prefix_len, prev_len, rtc_config):
    """Per-step correction weights of the guidance update, fp32 [steps,
    n_action_steps]: cw[k][r] = -dt * gw_k * w_r for the first prev_len
    positions, 0 after them (they have no previous action)
    (_predict_action_guidance_rtc, pi0_flowmatching.py:671-700;
    apply_rtc_guidance, rtc_guidance.py:107-155)."""
    w = compute_prefix_weights(n_action_steps, prefix_len,
                               rtc_config.get('decay_end', prefix_len * 2),
                               rtc_config.get('schedule', 'exp')).double()
    w[prev_len:] = 0.0
    max_gw = rtc_config.get('max_guidance_weight', 5.0)
    return torch.stack([-dt * compute_guidance_weight(1.0 - time, max_gw) * w
                        for time in times]).float()


def guidance_vjp_tables(times, n_action_steps, prefix_len, prev_len,
                        rtc_config):
    """Device tables of the guidance update with use_vjp: the prefix weights
    w (fp32 [n_action_steps], zero from prev_len on: those positions have no
    previous action) and each step's guidance weight gw (fp32 [steps])
    (_predict_action_guidance_rtc, pi0_flowmatching.py:671-700;
    rtc_guidance.py:28-104)."""
    w = compute_prefix_weights(n_action_steps, prefix_len,
                               rtc_config.get('decay_end', prefix_len * 2),
                               rtc_config.get('schedule', 'exp'))
    w[prev_len:] = 0.0
    max_gw = rtc_config.get('max_guidance_weight', 5.0)
    gw = torch.tensor([compute_guidance_weight(1.0 - time, max_gw)
                       for time in times], dtype=torch.float32)
    return w, gw
