"""PI0 action-chunk latency on one MI355X (BASELINE.json metric).

Workload (BASELINE config 4 at bs=1): 3 camera views of 224x224 uniform-noise
images + 48 random prompt tokens -> SigLIP-So400m/14 (27 layers) -> Gemma-2B
prefix (18 layers, 816 tokens) -> 10 Euler flow-matching steps of the
18-layer Gemma-300M action expert against the cached prefix K/V; output the
50 x 32 action chunk.  bf16 random-init weights (seeded), synthetic inputs.
One step = one whole chunk: input staging (copy_ into the static buffers)
plus one HIP graph replay.

Also reported on the same JSON line:
  roofline      the chunk's largest kernel by time (the bs=1 expert's decode
                attention, latency-bound, judged against HBM) timed live with
                HIP events on the stream it runs on, as in the chunk;
  roofline_mfma the largest MFMA-bound kernel (prefix GeGLU GEMM) the same
                way, weights cycled over the 17 layers, next to hipBLASLt
                on a plain GEMM of the same flops;
  kernels       the same for every main kernel of the chunk (and the C1
                RMSNorm+residual op), HBM-bound ones over distinct operand
                sets so that they do not run from the memory-side cache;
  phases        C2 (one expert layer, bs=1) and C3 (prefix prefill, bs=1)
                as HIP graphs of the chunk's kernels;
  cpu_baseline  the CPU oracle (fp32 restatement of the reference's eager
                PyTorch path) timed on this host: 1 warm-up + median of 3
                chunks, and config 1 alone (median of 20);
  configs       BASELINE configs 4 and 5 (ms/chunk, actions/s, accuracy);
  rtc           the same chunk with real-time chunking (prefix and guidance
                methods, guidance also with use_vjp, previous chunk of 30
                rows, prefix 5);
  serving       one predict_action request through the serving boundary
                (three 480x640 JPEG frames, msgpack): host decode, device
                preprocessing + chunk + device-to-host, reply encoding;
  parity        max abs error of the GPU chunk vs that CPU chunk.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = 'PI0 action-chunk latency ms @bs1 (10 flow steps); kernel % of HBM/MFMA peak'
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def log(msg):
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


TRAFFIC_PROFILE = os.path.join(ROOT, 'profiles', 'pi0_bs1_kernel_table_traffic.md')


def measured_traffic(row=None):
    """HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated)
    of a kernel-table row from the committed profile, keyed by row name
    (all rows if ``row`` is None); None where absent."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None if row is not None else {}
    out = {}
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip('|').split('|')]
        if len(cells) < 6:
            continue
        try:
            out[cells[0]] = int(round((float(cells[4]) + float(cells[5])) * 1e6))
        except ValueError:
            continue
    return out if row is None else out.get(row)


def _expert_attention_calls(model):
    """The chunk's expert decode attention launches at bs=1, one per layer:
    that layer's key / value cache, the chunk's prefetch list (the layer's
    weights and the next layer's cache) and the fragment-major output only,
    as _expert_layer_pi0_frag issues them."""
    from fluxvla_amd import kernels as K
    cfg = model.cfg
    b = model._bufs[1]
    S, Ss = cfg.prefix_len, cfg.suffix_len
    ctxf = b['ex_ctxf'].rows(Ss)
    calls = []
    for i in range(len(model.exp_f)):
        kc, vc = b['kc'][i], b['vc'][i]
        calls.append(lambda i=i, kc=kc, vc=vc: K.mqa_attention(
            b['ex_q'], kc[:, :S + Ss], vc, b['ex_ctx'], kgrp=b['kgrp'],
            qgrp=b['qgrp_suf'], v_transposed=True, o_frag=ctxf,
            o_row_major=False, prefetch=model._prefetch_list(i),
            prefetch_place=model.prefetch_place))
    return calls


def time_dominant_kernel(model, reps=20):
    """The chunk's largest kernel by time (rocprofv3 kernel trace of the
    chunk, profiles/pi0_bs1_chunk_kernel_stats.md): attn_decode_kernel, the
    bs=1 expert's decode attention (408 query rows = 51 tokens x 8 heads
    against 867 cached keys, 14 key ranges merged inside the launch, its
    idle workgroups prefetching the next GEMMs' weights), 180 launches per
    chunk.  Timed as in the chunk: the 18 layers' launches (each with its
    layer's cache and prefetch list) in one HIP graph, replayed between HIP
    events on the stream it runs on; the average per launch keeps the
    graph's kernel boundary, as the trace's durations do.  It is latency
    bound (timestamps inside the kernel: the query rows land ~3 us after the
    start, one tile's softmax and P V take ~2.5 us, the merge ~3.5 us);
    its roofline is HBM against its algorithmic bytes: the K and V rows of
    the 867 visible keys and Q and O (408 x 256 bf16 each), 1.31 MB."""
    cfg = model.cfg
    calls = _expert_attention_calls(model)
    us = _launch_time_us(calls, reps, min_calls=len(calls))
    T = cfg.prefix_len + cfg.suffix_len
    R = cfg.suffix_len * cfg.heads
    nbytes = 2 * T * cfg.head_dim * 2 + 2 * R * cfg.head_dim * 2
    achieved = nbytes / (us * 1e-6) / 1e9
    return {
        'kernel': 'attn_decode_kernel (expert decode attention + in-launch '
                  f'merge + weight prefetch, {R} query rows x {T} keys, '
                  'hd 256, 14 key ranges)',
        'bound': 'hbm',
        'achieved': round(achieved, 1),
        'peak': PEAK_HBM_GBS,
        'unit': 'GB/s',
        'frac': round(achieved / PEAK_HBM_GBS, 4),
        'traffic': measured_traffic('attn_decode_kernel + merge (expert)'),
        'traffic_unit': 'bytes/launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, '
                        'profiles/pi0_bs1_kernel_table_traffic.md; the '
                        'table row runs without the weight prefetch)',
        'avg_us': round(us, 2),
        'bytes_per_launch': nbytes,
        'launches_per_chunk': cfg.exp_layers * cfg.num_steps,
    }


def time_mfma_kernel(model, reps=10):
    """The chunk's largest MFMA-bound kernel: the prefix GeGLU GEMM
    (gemm_wide_kernel<GEGLU>, M=816, K=2048, N=16384 x 2 weights, rownorm
    with the row sums handed over by the O projection), 17 launches per
    chunk.  Timed as in the chunk: one launch per prefix layer with that
    layer's weights (17 x 134 MB, so each launch reads its weights from
    HBM), in a HIP graph replayed between HIP events.  ``library_us``: the
    vendor library (hipBLASLt through torch.matmul) on a plain GEMM of the
    same flops (x @ [Wg; Wu]^T, no epilogue), timed the same way."""
    import torch

    from fluxvla_amd import kernels as K
    cfg = model.cfg
    b = model._bufs[1]
    x = b['pre_x'].view(-1, cfg.llm_hidden)
    h = b['pre_h']
    ss = b['pre_ss'][0]
    layers = model.llm['layers'][:cfg.llm_layers - 1]
    calls = [lambda L=L: K.gemm_geglu(x, L['gate_w'], L['up_w'], out=h,
                                      rownorm_eps=cfg.rms_eps, ss_in=ss)
             for L in layers]
    us = _launch_time_us(calls, reps, min_calls=len(calls))
    M, N, Kd = x.shape[0], layers[0]['gate_w'].shape[0], x.shape[1]
    flops = 2.0 * M * N * Kd * 2
    achieved = flops / (us * 1e-6) / 1e12
    # the library on the same flops: [816, 2048] x [2048, 32768], 4 weight
    # sets (537 MB) cycled so that it also reads its weights from HBM
    g = torch.Generator(device=x.device).manual_seed(5)
    ws = [(torch.randn(2 * N, Kd, device=x.device, generator=g) * 0.02).bfloat16()
          for _ in range(4)]
    out = torch.empty(M, 2 * N, device=x.device, dtype=torch.bfloat16)
    lib_us = _launch_time_us([lambda w=w: torch.matmul(x, w.t(), out=out)
                              for w in ws], reps, min_calls=8)
    del ws
    return {
        'kernel': 'gemm_wide_kernel<GEGLU> (prefix gate/up, '
                  f'M={M} N={N}x2 K={Kd}, 17 layers\' weights cycled)',
        'bound': 'mfma',
        'achieved': round(achieved, 2),
        'peak': PEAK_BF16_TFLOPS,
        'unit': 'TFLOP/s',
        'frac': round(achieved / PEAK_BF16_TFLOPS, 4),
        'traffic': measured_traffic('gemm_wide_kernel<GEGLU> (prefix)'),
        'traffic_unit': 'bytes/launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, '
                        'profiles/pi0_bs1_kernel_table_traffic.md)',
        'avg_us': round(us, 2),
        'flops_per_launch': flops,
        'library_us': round(lib_us, 2),
        'library': 'hipBLASLt (torch.matmul), plain GEMM of the same flops, '
                   'no epilogue',
    }


def _graph_time_us(fn, reps=20):
    """Average us per replay of a HIP graph holding one call of ``fn``."""
    import torch
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        fn()
        torch.cuda.synchronize()
        g.capture_begin()
        fn()
        g.capture_end()
    torch.cuda.current_stream().wait_stream(st)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(
        enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / reps


def _launch_time_us(calls, reps, min_calls=16):
    """Average us per call: ``calls`` (distinct operand sets, so HBM-bound
    kernels are not served from the 256 MB memory-side cache; repeated to
    at least ``min_calls``) captured back to back in one HIP graph and
    replayed ``reps`` times between HIP events.  The graph keeps host launch
    overhead out of the figure; the ~1.6 us a kernel boundary costs inside a
    graph stays in it."""
    seq = list(calls) * max(1, -(-min_calls // len(calls)))

    def run():
        for c in seq:
            c()
    return _graph_time_us(run, reps) / len(seq)


def _row(name, shape, bound, work, us):
    if bound == 'hbm':
        achieved = work / (us * 1e-6) / 1e9
        peak, unit = PEAK_HBM_GBS, 'GB/s'
    else:
        achieved = work / (us * 1e-6) / 1e12
        peak, unit = PEAK_BF16_TFLOPS, 'TFLOP/s'
    # HBM bytes per launch from the committed rocprofv3 counter passes
    return {'kernel': name, 'shape': shape, 'bound': bound,
            'avg_us': round(us, 2), 'achieved': round(achieved, 1),
            'peak': peak, 'unit': unit, 'frac': round(achieved / peak, 4),
            'work': work, 'traffic': measured_traffic(name)}


def kernel_table(model):
    """Per-kernel rooflines at the chunk's shapes (algorithmic bytes or
    flops per launch / average launch time).  M = 51 GEMMs, norms and the
    decode attention are judged against HBM, M >= 768 GEMMs and prefill
    attention against bf16 MFMA.  HBM-bound kernels cycle through distinct
    operand sets (C1: 32 sets, 537 MB; expert: the 18 layers' weights,
    623 MB) so that the figures are HBM, not memory-side-cache, figures."""
    import torch

    from fluxvla_amd import kernels as K
    cfg, dev = model.cfg, model.device
    rows = []
    # C1: fused RMSNorm + residual, [1024, 2048]
    g = torch.Generator(device=dev).manual_seed(0)
    sets = []
    for _ in range(32):
        x = torch.randn(1024, 2048, device=dev, generator=g).bfloat16()
        r = torch.randn(1024, 2048, device=dev, generator=g).bfloat16()
        sets.append((x, r, torch.empty_like(x), torch.empty_like(x)))
    w = (torch.randn(2048, device=dev, generator=g) * 0.02 + 1).bfloat16()
    calls = [lambda s=s: K.rms_norm_residual(s[0], s[1], w, 1e-6, out=s[2],
                                             residual_out=s[3])
             for s in sets]
    nbytes = 4 * 1024 * 2048 * 2 + 2048 * 2
    rows.append(_row('rms_norm_residual_kernel (C1)', '[1024, 2048]', 'hbm',
                     nbytes, _launch_time_us(calls, 10)))
    rows.append(_row('rms_norm_residual_kernel (C1, cache-resident)',
                     '[1024, 2048]', 'hbm', nbytes,
                     _launch_time_us(calls[:1], 20, min_calls=32)))
    # the floor for these bytes: a plain row copy kernel (fvx_copy_rows)
    # reading and writing the same 16.8 MB, over 32 operand sets
    big = [(torch.empty(2048, 2048, dtype=torch.bfloat16, device=dev),
            torch.empty(2048, 2048, dtype=torch.bfloat16, device=dev))
           for _ in range(32)]
    one = _launch_time_us([lambda t=t: K.copy_rows(t[0], t[1]) for t in big],
                          10)
    rows.append(_row('copy_rows_kernel, same bytes (C1 floor: an 8.4 MB -> '
                     '8.4 MB copy)', '[2048, 2048] bf16', 'hbm', nbytes, one))
    del sets, calls, big

    # action expert at bs=1, fragment-major operands as in the chunk
    b = model._bufs[1]
    S, Ss, D, hid = cfg.prefix_len, cfg.suffix_len, cfg.head_dim, cfg.exp_hidden
    T = model.kv_len
    x = b['ex_x'].view(Ss, hid)
    xf, ctxf, hf = (b['ex_xf'].rows(Ss), b['ex_ctxf'].rows(Ss),
                    b['ex_hf'].rows(Ss))
    H, mlp = cfg.heads, cfg.exp_mlp
    qkv, oc, ggl, dn, att = [], [], [], [], []
    for i, Lf in enumerate(model.exp_f):
        kc, vc = b['kc'][i], b['vc'][i]
        qkv.append(lambda Lf=Lf, kc=kc, vc=vc: K.gemm_qkv_rope(
            xf, Lf['qkv_w'], model.rope, b['pos_suf'], b['ex_q'].view(Ss, -1),
            kc.view(T, D)[S:], vc[:, :, S:], H, D, rownorm_eps=cfg.rms_eps,
            row_group=Ss, row_group_stride=T, v_ld=T))
        att.append(lambda kc=kc, vc=vc: K.mqa_attention(
            b['ex_q'], kc[:, :S + Ss], vc, b['ex_ctx'], kgrp=b['kgrp'],
            qgrp=b['qgrp_suf'], v_transposed=True, o_frag=ctxf,
            o_row_major=False))
        oc.append(lambda Lf=Lf: K.gemm(ctxf, Lf['o_w'], out=x, residual=x,
                                       c_frag=xf))
        ggl.append(lambda Lf=Lf: K.gemm_geglu(xf, Lf['gate_w'], Lf['up_w'],
                                              out=b['ex_h'],
                                              rownorm_eps=cfg.rms_eps,
                                              c_frag=hf))
        dn.append(lambda Lf=Lf: K.gemm(hf, Lf['down_w'], out=x, residual=x,
                                       c_frag=xf))
    nq = (H + 2) * D
    for name, calls, N, Kd, nb, extra in (
            ('gemm_skinny_kernel<QKV_ROPE> (expert)', qkv, nq, hid, 1, 0),
            ('gemm_skinny_kernel<PLAIN> o-proj (expert)', oc, hid, H * D, 1,
             Ss * hid * 2),
            ('gemm_skinny_kernel<GEGLU> (expert)', ggl, mlp, hid, 2, 0),
            ('gemm_skinny_kernel<PLAIN> down (expert)', dn, hid, mlp, 1,
             Ss * hid * 2)):
        work = nb * N * Kd * 2 + Ss * Kd * 2 + Ss * N * 2 + extra
        rows.append(_row(name, f'M={Ss} N={N}{"x2" if nb == 2 else ""} K={Kd}',
                         'hbm', work, _launch_time_us(calls, 5)))
    T_keys = S + Ss
    work = T_keys * D * 2 * 2 + 2 * Ss * H * D * 2
    rows.append(_row('attn_decode_kernel + merge (expert)',
                     f'{Ss * H} query rows x {T_keys} keys', 'hbm', work,
                     _launch_time_us(att, 5)))

    # prefix (M = 816) and SigLIP (M = 768) GEMMs, prefill attention: MFMA;
    # each row cycles the layers' weights (17 prefix layers, 27 SigLIP
    # layers), as the chunk reads them: one launch per layer, from HBM
    px = b['pre_x'].view(-1, cfg.llm_hidden)
    M = px.shape[0]
    kc0, vc0 = b['kc'][0], b['vc'][0]
    # as in the chunk: the residual GEMMs hand the row sums of squares of x
    # to the next fused RMSNorm
    ss_a, ss_b = b['pre_ss'][0], b['pre_ss'][1]
    pre = [
        ('gemm_tile_kernel<64,128,QKV_ROPE> (prefix)', lambda L: K.gemm_qkv_rope(
            px, L['qkv_w'], model.rope, b['pos_pre'], b['pre_q'].view(M, -1),
            kc0.view(T, D), vc0, H, D, rownorm_eps=cfg.rms_eps, row_group=S,
            row_group_stride=T, v_ld=T, ss_in=ss_b), 2 * M * nq * cfg.llm_hidden),
        ('gemm_tile_kernel<64,128,PLAIN> o-proj (prefix)', lambda L: K.gemm(
            b['pre_ctx'].view(M, -1), L['o_w'], out=b['pre_h'][:, :cfg.llm_hidden],
            residual=px, ss_out=ss_a), 2 * M * cfg.llm_hidden * H * D),
        ('gemm_wide_kernel<GEGLU> (prefix)', lambda L: K.gemm_geglu(
            px, L['gate_w'], L['up_w'], out=b['pre_h'], rownorm_eps=cfg.rms_eps,
            ss_in=ss_a), 4 * M * cfg.llm_mlp * cfg.llm_hidden),
        ('gemm_wide_kernel<PLAIN> 8 K ranges + split-K reduce, down (prefix)', lambda L: K.gemm(
            b['pre_h'], L['down_w'], out=b['pre_q'].view(M, -1)[:, :cfg.llm_hidden],
            residual=px, ss_out=ss_b), 2 * M * cfg.llm_hidden * cfg.llm_mlp),
        ('attn_decode_t_kernel + merge (prefix)', lambda L: K.mqa_attention(
            b['pre_q'], kc0[:, :S], vc0, b['pre_ctx'], kgrp=b['kgrp'][:, :S],
            qgrp=b['qgrp_pre'], v_transposed=True), 4 * H * S * S * D),
    ]
    pre = [(n, f, fl, model.llm['layers'][:cfg.llm_layers - 1])
           for n, f, fl in pre]
    vx, vxn = b['vis_x'], b['vis_xn']
    Mv, vh = vx.shape
    nimg = Mv // cfg.num_patches
    vis = [
        ('gemm_tile_kernel<64,128,PLAIN> qkv+bias (SigLIP)', lambda V: K.gemm(
            vxn, V['qkv_w'], out=b['vis_qkv'], bias=V['qkv_b']),
         2 * Mv * 3 * vh * vh),
        ('gemm_tile_kernel<64,64,PLAIN> o-proj+bias+res (SigLIP)',
         lambda V: K.gemm(b['vis_ctx'], V['o_w'], out=vxn, bias=V['o_b'],
                        residual=vx), 2 * Mv * vh * vh),
        ('gemm_tile_kernel<64,128,PLAIN> fc1+bias+gelu (SigLIP)', lambda V: K.gemm(
            vxn, V['fc1_w'], out=b['vis_h'], bias=V['fc1_b'], act=2),
         2 * Mv * cfg.vit_mlp * vh),
        ('gemm_tile_kernel<64,64,PLAIN> fc2+bias+res (SigLIP)', lambda V: K.gemm(
            b['vis_h'], V['fc2_w'], out=vxn, bias=V['fc2_b'], residual=vx),
         2 * Mv * vh * cfg.vit_mlp),
        ('attn_kernel<96,80> (SigLIP)', lambda V: K.mha_packed_qkv(
            b['vis_qkv'], b['vis_ctx'], nimg, cfg.num_patches, cfg.vit_heads,
            cfg.vit_head_dim),
         4 * nimg * cfg.vit_heads * cfg.num_patches ** 2 * cfg.vit_head_dim),
    ]
    pre += [(n, f, fl, model.vis['layers']) for n, f, fl in vis]
    for name, fn, flops, layers in pre:
        calls = [lambda L=L, fn=fn: fn(L) for L in layers]
        rows.append(_row(name, '', 'mfma', flops,
                         _launch_time_us(calls, 5, min_calls=len(calls))))
    return rows


def phase_times(model):
    """C2 (one expert layer, one flow step, bs=1) and C3 (prefix prefill,
    bs=1) as HIP graphs of the chunk's own kernels."""
    b = model._bufs[1]
    c3 = _graph_time_us(lambda: (model.vision_encoder(b, 1),
                                 model.transformer_encoder(b, 1)), reps=10)
    L = model.exp['layers'][0]
    c2 = _graph_time_us(lambda: model._expert_layer_pi0(b, 1, 0, L), reps=50)
    return {'C2_expert_layer_bs1_us': round(c2, 2),
            'C3_prefix_prefill_bs1_ms': round(c3 / 1000.0, 3)}


def kernel_only(iters=10):
    """The dominant kernel alone at its chunk shape (random operands), then
    a plain 256 MiB device copy: the short program the rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE passes run (the copy calibrates the counters:
    it fetches and writes exactly 256 MiB)."""
    import torch

    from fluxvla_amd import kernels as K
    from fluxvla_amd.config import PI0
    cfg = PI0
    dev = torch.device('cuda', 0)
    g = torch.Generator(device=dev).manual_seed(0)
    M, Kd, N = cfg.prefix_len, cfg.llm_hidden, cfg.llm_mlp
    x = torch.randn(M, Kd, device=dev, generator=g).bfloat16()
    wg = (torch.randn(N, Kd, device=dev, generator=g) * 0.02).bfloat16()
    wu = (torch.randn(N, Kd, device=dev, generator=g) * 0.02).bfloat16()
    h = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    # the row sums of squares the O projection hands over in the chunk
    ss = x.float().view(M, -1, 64).pow(2).sum(-1).t().contiguous()
    for _ in range(iters):
        K.gemm_geglu(x, wg, wu, out=h, rownorm_eps=cfg.rms_eps, ss_in=ss)
    torch.cuda.synchronize()
    src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f'kernel-only: {iters} x gemm_geglu M={M} N={N}x2 K={Kd}; '
        '3 x copy 256 MiB')


def calibration_copy(nbytes=256 << 20, reps=3):
    """A plain device copy of known size: it fetches and writes exactly
    ``nbytes`` per dispatch, which calibrates rocprofv3's FETCH_SIZE /
    WRITE_SIZE counters."""
    import torch
    src = torch.ones(nbytes, dtype=torch.uint8, device='cuda')
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()


def table_only():
    """The per-kernel table alone (bs=1 PI0 model, one chunk first so the
    buffers hold chunk data), then the calibration copy: the program the
    rocprofv3 kernel-trace and FETCH_SIZE / WRITE_SIZE passes run."""
    import torch

    from fluxvla_amd.config import PI0
    from fluxvla_amd.pi0_inference import PI0Inference
    from fluxvla_amd.weights import make_inputs, make_state_dict
    dev = torch.device('cuda', 0)
    sd = make_state_dict(PI0, seed=0, device=dev)
    model = PI0Inference(PI0, sd, device=dev, max_batch=1)
    inp = {k: v.to(dev) for k, v in make_inputs(PI0, batch=1, seed=1).items()}
    model.predict_action(inp['images'], inp['lang_tokens'], inp['states'],
                         inp['img_masks'], inp['lang_masks'],
                         noise=inp['noise'])
    torch.cuda.synchronize()
    rows = kernel_table(model)
    for r in rows:
        log(f"  {r['kernel']:56s} {r['avg_us']:9.2f} us "
            f"{r['achieved']:8.1f} {r['unit']} ({100 * r['frac']:.1f} %)")
    calibration_copy()
    log('table-only: done (last dispatches: 3 x copy 256 MiB)')
    print(json.dumps({'kernels': rows}), flush=True)


# ---------------------------------------------------------------------------
# rocprofv3 summaries: profiles/*.md from the CSVs of four profiler passes
# ---------------------------------------------------------------------------
# (output directory, -o prefix, profiler options, bench.py options)
PROFILE_PASSES = (
    ('ptab_kt', 'kt', '--kernel-trace --stats', '--table-only'),
    ('ptab_fetch', 'fetch', '--pmc FETCH_SIZE', '--table-only'),
    ('ptab_write', 'write', '--pmc WRITE_SIZE', '--table-only'),
    ('pvjp', 'vjp', '--kernel-trace --stats', '--vjp-only'),
    ('pbench', 'bench', '--kernel-trace --stats', ''),
)


def _profile_command(name):
    """profile_commands()'s line of the pass writing into ``name``."""
    names = [d for d, _, _, _ in PROFILE_PASSES]
    return profile_commands()[names.index(name)]


def profile_commands(out='$R/gpurun_out'):
    """The profiler commands whose CSVs summarize_profiles reads (repo root
    ``R``; TMPDIR=/tmp), one line each."""
    cmds = []
    for d, o, opts, args in PROFILE_PASSES:
        cmds.append(f'rocprofv3 {opts} --output-format csv -d {out}/{d} -o {o} '
                    f'-- python3 $R/bench.py{" " + args if args else ""}'
                    f' > {out}/{d}.log 2>&1')
    return cmds


def _kernel_name(full):
    """A kernel's name without its argument list (and without the
    '(anonymous namespace)::' scope, whose parenthesis is not one)."""
    return (full.replace('void ', '').replace('(anonymous namespace)::', '')
            .split('(')[0])


def _trace(path):
    """Kernel-trace CSV rows in start order with name, workgroups, us."""
    import csv
    rows = sorted(csv.DictReader(open(path)),
                  key=lambda r: int(r['Start_Timestamp']))
    for r in rows:
        r['name'] = _kernel_name(r['Kernel_Name'])
        wg = 1
        for ax in 'XYZ':
            wg *= max(1, int(r.get(f'Grid_Size_{ax}', 1)) //
                      max(1, int(r.get(f'Workgroup_Size_{ax}', 1))))
        r['wgs'] = wg
        r['us'] = (int(r['End_Timestamp']) - int(r['Start_Timestamp'])) / 1e3
    return rows


def _counters(path):
    """Counter-collection CSV rows in dispatch order: (name, wgs, KiB)."""
    import csv
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r['Dispatch_Id']))
    return [(_kernel_name(r['Kernel_Name']),
             int(r['Grid_Size']) // max(1, int(r['Workgroup_Size'])),
             float(r['Counter_Value'])) for r in rows]


def _after_last(seq, name_of, sub):
    """The entries after the last one whose name contains ``sub``."""
    idx = [i for i, x in enumerate(seq) if sub in name_of(x)]
    return seq[idx[-1] + 1:] if idx else seq


def _json_line(path):
    line = None
    for s in open(path):
        if s.startswith('{'):
            line = s
    return json.loads(line) if line else None


# the per-kernel table's rows as dispatched by kernel_table (in order):
# (row, [(kernel-name substring, workgroups, dispatches), ...]); dispatches =
# one eager call + 3 warm-up + the timed graph replays, per operand set
_E, _MP, _MV = 18 * 9, 17 * 9, 27 * 9
TABLE_DISPATCHES = (
    # C1: 2048-column rows take one 4-wave workgroup each
    ('rms_norm_residual_kernel (C1)', [('rms_norm_residual_kernel', 1024, 32 * 14)]),
    ('rms_norm_residual_kernel (C1, cache-resident)',
     [('rms_norm_residual_kernel', 1024, 32 * 24)]),
    ('copy_rows_kernel, same bytes (C1 floor: an 8.4 MB -> 8.4 MB copy)',
     [('copy_rows_kernel', 2048, 32 * 14)]),
    ('gemm_skinny_kernel<QKV_ROPE> (expert)', [('gemm_skinny_kernel<2', 160, _E)]),
    ('gemm_skinny_kernel<PLAIN> o-proj (expert)', [('gemm_skinny_kernel<0', 256, _E)]),
    ('gemm_skinny_kernel<GEGLU> (expert)', [('gemm_skinny_kernel<1', 256, _E)]),
    ('gemm_skinny_kernel<PLAIN> down (expert)', [('gemm_skinny_kernel<0', 256, _E)]),
    ('attn_decode_kernel + merge (expert)', [('attn_decode_kernel', 176, _E)]),
    ('gemm_tile_kernel<64,128,QKV_ROPE> (prefix)',
     [('gemm_tile_kernel<64, 128, 2, 2, 3, 2', 260, _MP)]),
    ('gemm_tile_kernel<64,128,PLAIN> o-proj (prefix)',
     [('gemm_tile_kernel<64, 128, 2, 2, 4, 0', 208, _MP)]),
    ('gemm_wide_kernel<GEGLU> (prefix)', [('gemm_wide_kernel<1', 512, _MP)]),
    ('gemm_wide_kernel<PLAIN> 8 K ranges + split-K reduce, down (prefix)',
     [('gemm_wide_kernel<0', 256, _MP), ('gemm_partial_reduce_kernel<0', 816, _MP)]),
    ('attn_decode_t_kernel + merge (prefix)',
     [('attn_decode_t_kernel', 204, _MP), ('attn_decode_merge_kernel', 816, _MP)]),
    ('gemm_tile_kernel<64,128,PLAIN> qkv+bias (SigLIP)',
     [('gemm_tile_kernel<64, 128, 2, 2, 3, 0', 324, _MV)]),
    ('gemm_tile_kernel<64,64,PLAIN> o-proj+bias+res (SigLIP)',
     [('gemm_tile_kernel<64, 64, 2, 2, 4, 0', 216, _MV)]),
    ('gemm_tile_kernel<64,128,PLAIN> fc1+bias+gelu (SigLIP)',
     [('gemm_tile_kernel<64, 128, 2, 2, 3, 0', 408, _MV)]),
    ('gemm_tile_kernel<64,64,PLAIN> fc2+bias+res (SigLIP)',
     [('gemm_tile_kernel<64, 64, 2, 2, 4, 0', 216, _MV)]),
    ('attn_kernel<96,80> (SigLIP)', [('attn_kernel<96, 80>', 192, _MV)]),
)


def _runs(rows, sub, min_len):
    """Maximal runs of >= min_len consecutive dispatches of one kernel."""
    runs, cur = [], []
    for r in rows + [None]:
        if r is not None and sub in r['name']:
            cur.append(r)
            continue
        if len(cur) >= min_len:
            runs.append(cur)
        cur = []
    return runs


def _run_line(run):
    import statistics
    d = [r['us'] for r in run]
    span = (int(run[-1]['End_Timestamp']) -
            int(run[0]['Start_Timestamp'])) / 1e3 / len(run)
    return (f'{len(run)} dispatches: mean {statistics.mean(d):.2f} us, median '
            f'{statistics.median(d):.2f}, min {min(d):.2f}, max {max(d):.2f}, '
            f'span/launch {span:.2f} us')


def summarize_profiles(gdir, outdir):
    """Write profiles/pi0_bs1_kernel_table_traffic.md,
    pi0_bs1_chunk_kernel_stats.md and pi0_bs1_dominant_kernel_trace.md
    into ``outdir`` from the CSVs the PROFILE_PASSES commands left under
    ``gdir`` (and the JSON lines those runs printed to their logs)."""
    import statistics
    os.makedirs(outdir, exist_ok=True)
    cmds = '\n'.join('    ' + c for c in profile_commands())
    # ---- per-kernel table: durations and calibrated traffic ----
    name0 = lambda x: x[0]  # noqa: E731
    kt = [(r['name'], r['wgs'], r['us'])
          for r in _trace(f'{gdir}/ptab_kt/kt_kernel_trace.csv')]
    # the table's dispatches follow the chunk run first (its last Euler GEMM)
    kt = _after_last(kt, name0, 'gemm_skinny_kernel<3')
    fe = _after_last(_counters(f'{gdir}/ptab_fetch/fetch_counter_collection.csv'),
                     name0, 'gemm_skinny_kernel<3')
    wr = _after_last(_counters(f'{gdir}/ptab_write/write_counter_collection.csv'),
                     name0, 'gemm_skinny_kernel<3')
    # calibration: the three 256 MiB copies at the end of the program
    cf = statistics.median([v for n, w, v in fe if 'copyBuffer' in n][-3:])
    cw = statistics.median([v for n, w, v in wr if 'copyBuffer' in n][-3:])
    sf, sw = 262144 / cf, 262144 / cw
    bench_rows = {r['kernel']: r for r in
                  (_json_line(f'{gdir}/ptab_kt.log') or {}).get('kernels', [])}
    used = {}

    def take(seq, tag, sub, wg, cnt):
        idx = [i for i, x in enumerate(seq) if sub in x[0] and x[1] == wg]
        start = used.get((tag, sub, wg), 0)
        used[(tag, sub, wg)] = start + cnt
        return [seq[i][2] for i in idx[start:start + cnt]]
    lines = []
    for row, parts in TABLE_DISPATCHES:
        tt = tf = tw = 0.0
        descr, nmin = [], None
        for sub, wg, cnt in parts:
            t = take(kt, 'kt', sub, wg, cnt)
            f = take(fe, 'fe', sub, wg, cnt)
            w = take(wr, 'wr', sub, wg, cnt)
            if not (t and f and w):
                continue
            tt += statistics.median(t)
            tf += statistics.median(f) * sf * 1024 / 1e6
            tw += statistics.median(w) * sw * 1024 / 1e6
            base = sub.split('<')[0]
            descr.append(f'`{base}{"<..>" if "<" in sub else ""}` ({wg})')
            nmin = len(t) if nmin is None else min(nmin, len(t))
        b = bench_rows.get(row)
        ratio = (f'{(tf + tw) * 1e6 / b["work"]:.2f}'
                 if b and b['bound'] == 'hbm' else '')
        lines.append(f'| {row} | {" + ".join(descr)} | {nmin} | {tt:.2f} | '
                     f'{tf:.2f} | {tw:.2f} | {ratio} |')
    with open(f'{outdir}/pi0_bs1_kernel_table_traffic.md', 'w') as fh:
        fh.write(f"""# PI0 bs=1 per-kernel table -- rocprofv3 durations and HBM traffic

Every row of bench.py's per-kernel table (each main kernel of the chunk at
its chunk shape; every row cycles the layers' operands, as the chunk reads
them), with its rocprofv3 kernel duration and its calibrated FETCH_SIZE /
WRITE_SIZE bytes per dispatch.

Commands (repo root `R` on the MI355X box, `export TMPDIR=/tmp`; the first
three passes run the same program, one counter block each; this file is
`python3 bench.py --summarize-profiles gpurun_out` over their CSVs):

{cmds}

`bench.py --table-only` runs one chunk, then the table, then three copies of
256 MiB.  Calibration (a device copy fetches and writes exactly its size):
the copy reads FETCH {cf:.0f} KiB and WRITE {cw:.0f} KiB per dispatch, so
FETCH is scaled by {sf:.3f} and WRITE by {sw:.3f}.  The rows are the
table's own dispatches (those after the chunk), matched to the table rows
in order; durations are the kernel-trace pass's median per row (the counter
passes serialize dispatches, so their durations are not used); bytes are
the counter medians times the calibration factors.  "traffic /
algorithmic" = (FETCH + WRITE) / the row's algorithmic bytes (bench.py's
`work`) for the HBM-bound rows.

| bench row | kernel (WGs) | dispatches | rocprof median us | FETCH MB | WRITE MB | traffic / algorithmic |
|---|---|---:|---:|---:|---:|---:|
""" + '\n'.join(lines) + '\n')

    # ---- the default bench run: one chunk of its timed loop ----
    rows = _trace(f'{gdir}/pbench/bench_kernel_trace.csv')
    js = _json_line(f'{gdir}/pbench.log') or {}
    att_runs = _runs(rows, 'attn_decode_kernel', 18)
    # the timed loop ends where the roofline timing's launches start
    stop = rows.index(att_runs[0][0]) if att_runs else len(rows)
    starts = [i for i in range(stop) if 'im2col_kernel' in rows[i]['name']]
    chunk = None
    for j, s0 in enumerate(starts):
        s1 = starts[j + 1] if j + 1 < len(starts) else stop
        ends = [i for i in range(s0, s1)
                if 'gemm_skinny_kernel<3' in rows[i]['name']]
        if ends:
            chunk = rows[s0:ends[-1] + 1]
    agg = {}
    for r in chunk:
        a = agg.setdefault(r['name'], [0, 0.0])
        a[0] += 1
        a[1] += r['us']
    tot = sum(a[1] for a in agg.values())
    span = (int(chunk[-1]['End_Timestamp']) -
            int(chunk[0]['Start_Timestamp'])) / 1e6
    table = '\n'.join(f'| `{n}` | {c} | {d / 1e3:.3f} | {d / c:.2f} |'
                      for n, (c, d) in sorted(agg.items(), key=lambda kv: -kv[1][1]))
    with open(f'{outdir}/pi0_bs1_chunk_kernel_stats.md', 'w') as fh:
        fh.write(f"""# PI0 bs=1 action chunk -- rocprofv3 kernel statistics

Command (repo root `R` on the MI355X box, `export TMPDIR=/tmp`; the default
bench run itself; this file is `python3 bench.py --summarize-profiles
gpurun_out` over its CSV):

    {_profile_command('pbench')}

The last whole chunk of bench.py's timed loop (graph replay; from its
im2col to its last Euler GEMM).  The same run printed value =
{js.get('value')} ms per chunk (its own HIP events around the graph
replays, slowed by the profiler tracing every dispatch; the kernel times
below are the trace's own).

One chunk: {len(chunk)} dispatches, {tot / 1e3:.3f} ms of kernel time over a
{span:.3f} ms span.

| kernel | calls | ms | avg us |
|---|---:|---:|---:|
{table}
""")

    # ---- the roofline kernels' own launches in the same run ----
    roof, mf = js.get('roofline') or {}, js.get('roofline_mfma') or {}
    att = '\n'.join('    ' + _run_line(r) for r in att_runs)
    geg = '\n'.join('    ' + _run_line(r)
                    for r in _runs(rows, 'gemm_wide_kernel<1', 17))
    with open(f'{outdir}/pi0_bs1_dominant_kernel_trace.md', 'w') as fh:
        fh.write(f"""# Roofline kernels of the PI0 bs=1 chunk -- rocprofv3 kernel trace of bench.py

`roofline`: the chunk's largest kernel by time, `attn_decode_kernel` (the
bs=1 expert's decode attention: 408 query rows x 867 keys, 14 key ranges
merged inside the launch, idle workgroups prefetching the next GEMMs'
weights and the next layer's key / value cache; {roof.get('bytes_per_launch')}
algorithmic bytes per launch, {roof.get('launches_per_chunk')} launches per
chunk).  `roofline_mfma`: the prefix GeGLU GEMM (`gemm_wide_kernel<1, ...>`,
M=816, N=16384 x 2, K=2048, {mf.get('flops_per_launch')} flops per launch).

Command (repo root `R` on the MI355X box, `export TMPDIR=/tmp`; the default
bench run; this file is `python3 bench.py --summarize-profiles gpurun_out`):

    {_profile_command('pbench')}

Runs of back-to-back dispatches in start order (durations End - Start;
span/launch = first start to last end over the run, which keeps the kernel
boundaries as bench.py's HIP-event figure does).  bench.py times the 18
expert layers' launches in one graph (one eager pass, then 3 + 20
replays): its run is the {18 * 23}-dispatch one.

attn_decode_kernel (bench.py in the same run: avg_us {roof.get('avg_us')} per
launch, frac {roof.get('frac')} of HBM peak):

{att}

gemm_wide_kernel<1> (bench.py: avg_us {mf.get('avg_us')}, {mf.get('achieved')}
TFLOP/s, frac {mf.get('frac')}; hipBLASLt on the same flops
{mf.get('library_us')} us):

{geg}
""")


def summarize_vjp_profile(gdir, outdir):
    """profiles/pi0_bs1_vjp_chunk_kernel_stats.md from the --vjp-only pass:
    the kernels of its last whole guidance-with-VJP chunk."""
    path = f'{gdir}/pvjp/vjp_kernel_trace.csv'
    if not os.path.exists(path):
        return
    rows = _trace(path)
    js = _json_line(f'{gdir}/pvjp.log') or {}
    starts = [i for i, r in enumerate(rows) if 'im2col_kernel' in r['name']]
    s0 = starts[-1]
    ends = [i for i in range(s0, len(rows)) if 'rtc_vjp_update' in rows[i]['name']]
    chunk = rows[s0:ends[-1] + 1]
    agg = {}
    for r in chunk:
        a = agg.setdefault(r['name'], [0, 0.0])
        a[0] += 1
        a[1] += r['us']
    tot = sum(a[1] for a in agg.values())
    span = (int(chunk[-1]['End_Timestamp']) -
            int(chunk[0]['Start_Timestamp'])) / 1e6
    table = '\n'.join(f'| `{n}` | {c} | {d / 1e3:.3f} | {d / c:.2f} |'
                      for n, (c, d) in sorted(agg.items(), key=lambda kv: -kv[1][1]))
    with open(f'{outdir}/pi0_bs1_vjp_chunk_kernel_stats.md', 'w') as fh:
        fh.write(f"""# PI0 bs=1 chunk with guidance RTC and use_vjp -- rocprofv3 kernel statistics

Command (repo root `R` on the MI355X box, `export TMPDIR=/tmp`; this file
is `python3 bench.py --summarize-profiles gpurun_out` over its CSV):

    {_profile_command('pvjp')}

`bench.py --vjp-only` builds the PI0 bs=1 model, then runs chunks with
guidance real-time chunking and use_vjp (a previous chunk of 30 rows,
prefix 5; each Euler step a forward with saved activations and a backward
through the expert) through their captured graph.  The last whole chunk
(from its im2col to its last guidance update).  The same run printed
{js.get('ms_per_chunk')} ms per chunk (wall clock over its timed chunks,
slowed by the profiler tracing every dispatch; the kernel times below are
the trace's own).

One chunk: {len(chunk)} dispatches, {tot / 1e3:.3f} ms of kernel time over a
{span:.3f} ms span.

| kernel | calls | ms | avg us |
|---|---:|---:|---:|
{table}
""")


def vjp_only(steps=5):
    """Guidance-with-VJP chunks alone (PI0 bs=1): the program of the
    rocprofv3 pass behind the VJP kernel statistics."""
    import torch

    from fluxvla_amd.config import PI0
    from fluxvla_amd.pi0_inference import PI0Inference
    from fluxvla_amd.weights import make_inputs, make_state_dict
    dev = torch.device('cuda', 0)
    sd = make_state_dict(PI0, seed=0, device=dev)
    model = PI0Inference(PI0, sd, device=dev, max_batch=1)
    dinp = {k: v.to(dev) for k, v in make_inputs(PI0, batch=1, seed=1).items()}
    g = torch.Generator().manual_seed(5)
    prev = (torch.randn(1, 30, 32, generator=g) * 0.5).to(dev)
    rc = {'enabled': True, 'method': 'guidance', 'use_vjp': True,
          'max_guidance_weight': 5.0}

    def step():
        return model.predict_action(dinp['images'], dinp['lang_tokens'],
                                    dinp['states'], dinp['img_masks'],
                                    dinp['lang_masks'], noise=dinp['noise'],
                                    prev_actions=prev, prefix_len=5,
                                    rtc_config=rc)
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    log(f'vjp-only: {ms:.3f} ms per chunk')
    print(json.dumps({'ms_per_chunk': round(ms, 3)}), flush=True)


def cpu_model_name():
    """The host CPU's model string (/proc/cpuinfo), else platform's guess."""
    import platform
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_c1_ms(reps=20):
    """BASELINE config 1 on the CPU: the fp32 PyTorch restatement of the
    residual add + GemmaRMSNorm (condition_gemma.py:75-116, :319-337) on
    x, residual [1024, 2048] bf16; median of ``reps`` runs after one
    warm-up."""
    import torch
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1024, 2048, generator=g).bfloat16()
    r = torch.randn(1024, 2048, generator=g).bfloat16()
    w = (torch.randn(2048, generator=g) * 0.02 + 1).bfloat16()

    def run():
        h = x.float() + r.float()
        y = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
        return y.bfloat16(), h.bfloat16()
    run()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        ts.append((time.perf_counter() - t0) * 1e3)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline(sd_gpu, cfg, inp, gpu_out, reps=3):
    """The CPU oracle (fp32 restatement of the reference's eager PyTorch
    path) on all host threads: one warm-up chunk, then the median of
    ``reps`` timed chunks of the same bs=1 request; and config 1 alone
    (median of 20).  Returns (cpu_baseline dict, GPU-vs-CPU chunk error)."""
    import torch

    from oracle import pi0_oracle
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    sd = {k: v.cpu() for k, v in sd_gpu.items()}

    def chunk():
        return pi0_oracle.predict_action(sd, cfg, inp['images'],
                                         inp['lang_tokens'], inp['states'],
                                         inp['img_masks'], inp['lang_masks'],
                                         inp['noise'])
    ref = chunk()  # warm-up
    runs = []
    for _ in range(reps):
        t0 = time.perf_counter()
        chunk()
        runs.append((time.perf_counter() - t0) * 1e3)
    err = (gpu_out.cpu() - ref).abs().max().item()
    med = sorted(runs)[len(runs) // 2]
    return {
        'value': round(med, 1),
        'unit': 'ms/chunk',
        'cores': n,
        'kind': 'port',
        'cpu_model': cpu_model_name(),
        'sample': f'full PI0 bs=1 chunk (prefix 816 + 10 steps), fp32 oracle: '
                  f'1 warm-up + median of {reps} chunks',
        'runs_ms': [round(t, 1) for t in runs],
        'c1_rms_norm_residual_ms': round(cpu_c1_ms(), 3),
    }, err


def time_chunks(model, cfg, batch, seed, warmup=2, steps=5):
    """Median HIP-event ms of ``steps`` graph-replayed chunks at ``batch``
    (inputs staged in HBM first, as for the headline figure)."""
    import torch

    from fluxvla_amd.weights import make_inputs
    dev = model.device
    inp = {k: v.to(dev) for k, v in make_inputs(cfg, batch=batch,
                                                seed=seed).items()}

    def step():
        return model.predict_action(inp['images'], inp['lang_tokens'],
                                    inp['states'], inp['img_masks'],
                                    inp['lang_masks'], noise=inp['noise'])
    for _ in range(warmup):
        out = step()
    torch.cuda.synchronize()
    per = []
    for _ in range(steps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        out = step()
        e1.record()
        e1.synchronize()
        per.append(e0.elapsed_time(e1))
    return sorted(per)[len(per) // 2], out, inp


def batch_accuracy(model, cfg, inp, out, samples, sd_ref=None,
                   oracle_samples=()):
    """Accuracy of a batched chunk ``out`` (inputs ``inp``): each listed
    sample against a bs=1 run of the same request through the same model
    (the skinny / tiled bs=1 kernels), and ``oracle_samples`` against the
    CPU oracle run with ``sd_ref`` (fp32, the weights the model applies)."""
    import torch
    res = {}
    worst = 0.0
    for s in samples:
        one = {k: v[s:s + 1] for k, v in inp.items()}
        o1 = model.predict_action(one['images'], one['lang_tokens'],
                                  one['states'], one['img_masks'],
                                  one['lang_masks'], noise=one['noise'])
        worst = max(worst, (out[s:s + 1] - o1).abs().max().item())
    res['max_abs_diff_vs_bs1_same_samples'] = worst
    res['samples'] = list(samples)
    if oracle_samples and sd_ref is not None:
        from oracle import pi0_oracle
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        worst = 0.0
        for s in oracle_samples:
            c = {k: v[s:s + 1].cpu() for k, v in inp.items()}
            r = pi0_oracle.predict_action(sd_ref, cfg, c['images'],
                                          c['lang_tokens'], c['states'],
                                          c['img_masks'], c['lang_masks'],
                                          c['noise'])
            worst = max(worst, (out[s:s + 1].cpu() - r).abs().max().item())
        res['max_abs_err_vs_cpu_oracle'] = worst
        res['oracle_samples'] = list(oracle_samples)
    return res


def other_configs(pi0_model, sd0, dev, parity=True):
    """BASELINE configs 4 (PI0 at bs 8) and 5 (PI0.5 with fp8 e4m3 weights
    in every Gemma-2B and expert linear, bs 1 / 8 / 32; W8A16 as the config
    states it, W8A8 as the opt-in variant), plus PI0.5 bf16 at bs 1 for
    reference.  Each: ms per chunk (median of 5 graph replays),
    actions/s and an accuracy figure: batched chunks against bs=1 runs of
    the same samples, and (with ``parity``) one sample per config against
    the CPU oracle (fp8: run on the dequantized weights; bars 2e-2 / 5e-2)."""
    import torch

    from fluxvla_amd.config import PI0, PI05
    from fluxvla_amd.pi0_inference import PI0Inference
    from fluxvla_amd.weights import make_state_dict
    rows = []

    def row(name, model_name, weights, batch, ms, cfg, acc=None, tol=None):
        r = {'config': name, 'model': model_name, 'weights': weights,
             'batch': batch, 'ms_per_chunk': round(ms, 3),
             'actions_per_s': round(batch * cfg.n_action_steps / ms * 1e3, 1)}
        if acc is not None:
            r['accuracy'] = dict(acc, tolerance=tol)
        log(f'  {name} {model_name} {weights} bs={batch}: {ms:.3f} ms/chunk'
            + (f' accuracy {acc}' if acc else ''))
        rows.append(r)

    sd0_cpu = {k: v.cpu() for k, v in sd0.items()} if parity else None
    ms, out, inp = time_chunks(pi0_model, PI0, 8, seed=21)
    acc = batch_accuracy(pi0_model, PI0, inp, out, (0, 7), sd0_cpu,
                         (0,) if parity else ())
    row('C4', 'PI0', 'bf16', 8, ms, PI0, acc, 2e-2)
    del sd0_cpu
    sd5 = make_state_dict(PI05, seed=0, device=dev)
    ref = PI0Inference(PI05, sd5, device=dev, max_batch=1)
    ms, _, _ = time_chunks(ref, PI05, 1, seed=22)
    row('C5-ref', 'PI0.5', 'bf16', 1, ms, PI05)
    del ref
    torch.cuda.empty_cache()
    parity_res = {}
    sd5_cpu = {k: v.cpu() for k, v in sd5.items()} if parity else None
    # W8A16 is config 5 as stated (bf16 activations, fp32 accumulate); W8A8
    # (activations quantized to e4m3 in the GEMMs) is the opt-in variant
    for wdt, label, tol in (('fp8', 'fp8_e4m3_w8a16', 2e-2),
                            ('fp8_w8a8', 'fp8_e4m3_w8a8', 5e-2)):
        fp8 = PI0Inference(PI05, sd5, device=dev, max_batch=32,
                           weight_dtype=wdt)
        sdq = fp8.dequantized_state_dict(sd5_cpu) if parity else None
        for batch in (1, 8, 32):
            ms, out, inp = time_chunks(fp8, PI05, batch, seed=23)
            if batch == 1:
                acc = batch_accuracy(fp8, PI05, inp, out, (), sdq,
                                     (0,) if parity else ())
                acc.pop('max_abs_diff_vs_bs1_same_samples')
                acc.pop('samples')
                if parity:
                    parity_res[label] = {
                        'chunk_max_abs_err_vs_cpu_oracle_dequantized':
                        acc['max_abs_err_vs_cpu_oracle'], 'tolerance': tol}
            else:
                acc = batch_accuracy(fp8, PI05, inp, out, (0, batch - 1), sdq,
                                     (0,) if parity and batch == 8 else ())
            row('C5', 'PI0.5', label, batch, ms, PI05, acc, tol)
        del fp8, sdq
        torch.cuda.empty_cache()
    del sd5, sd5_cpu
    torch.cuda.empty_cache()
    return rows, parity_res


def rtc_times(model, dinp, steps=10):
    """ms/chunk of the prefix and guidance RTC loops at bs=1 (each its own
    captured graph; guidance also with use_vjp: forward and backward through
    the expert at every step), and the locked rows' exactness."""
    import torch
    g = torch.Generator().manual_seed(5)
    prev = (torch.randn(1, 30, 32, generator=g) * 0.5).to(dinp['images'].device)
    out = {}
    for method in ('prefix', 'guidance', 'guidance_vjp'):
        rc = {'enabled': True, 'method': method.split('_')[0],
              'max_guidance_weight': 5.0,
              'use_vjp': method == 'guidance_vjp'}

        def step():
            return model.predict_action(dinp['images'], dinp['lang_tokens'],
                                        dinp['states'], dinp['img_masks'],
                                        dinp['lang_masks'], noise=dinp['noise'],
                                        prev_actions=prev, prefix_len=5,
                                        rtc_config=rc)
        for _ in range(2):
            a = step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            a = step()
        torch.cuda.synchronize()
        out[method] = {'ms_per_chunk': round((time.perf_counter() - t0) * 1e3 / steps, 3)}
        if method == 'prefix':
            out[method]['locked_rows_exact'] = bool(torch.equal(a[:, :5], prev[:, :5]))
    return out


def serving_latency(model, cfg, dinp, reps=10):
    """One predict_action request end to end through the serving boundary:
    three 480x640 uint8 frames JPEG-encoded in a msgpack request; the
    server decodes them (host), uploads the uint8 frames, preprocesses them
    on the GPU (ResizeImages + NormalizeImages of the PI0 aloha config),
    runs the chunk graph, copies the actions to the host and encodes the
    reply.  Medians over ``reps`` requests."""
    import numpy as np
    import torch

    from fluxvla_amd.preprocess import ImagePreprocessor
    from fluxvla_amd.serving import serializers as S
    from fluxvla_amd.serving.server import ObsToInputs, create_server
    cams = ['cam_high', 'cam_left_wrist', 'cam_right_wrist']
    g = torch.Generator().manual_seed(3)
    obs = {c: torch.randint(0, 256, (480, 640, 3), generator=g,
                            dtype=torch.uint8).numpy() for c in cams}
    obs['state'] = dinp['states'][0].cpu().numpy()
    obs['lang_tokens'] = dinp['lang_tokens'][0].cpu().numpy()
    obs['lang_masks'] = dinp['lang_masks'][0].cpu().numpy()
    means = [[123.515625, 116.04492188, 103.59375]] * 3
    stds = [[58.27148438, 57.02636719, 57.27539062]] * 3
    pre = ImagePreprocessor.from_transforms([
        dict(type='ResizeImages', height=224, width=224),
        dict(type='NormalizeImages', means=means, stds=stds)])
    ds = ObsToInputs(cams, pre, device=dinp['images'].device,
                     state_dim=cfg.state_dim)
    srv = create_server(model, dataset=ds, device=str(dinp['images'].device),
                        bind=False)
    req = S.encode_predict_request(obs, '')
    dec, handle, infer = [], [], []
    for i in range(reps + 2):
        t0 = time.perf_counter()
        S.decode_predict_request(req)
        t1 = time.perf_counter()
        resp = S.decode_predict_response(srv.handle(req))
        t2 = time.perf_counter()
        if i >= 2:
            dec.append((t1 - t0) * 1e3)
            handle.append((t2 - t1) * 1e3)
            infer.append(resp['infer_time'] * 1e3)
    # the preprocessing kernels alone (3 views), HIP events
    views = [torch.from_numpy(obs[c])[None].to(dinp['images'].device) for c in cams]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    pre(views)
    e0.record()
    for _ in range(20):
        pre(views)
    e1.record()
    torch.cuda.synchronize()
    med = lambda v: round(float(np.median(v)), 3)  # noqa: E731
    return {'request_ms': med(handle), 'host_decode_ms': med(dec),
            'predict_action_ms': med(infer),
            'gpu_preprocess_us': round(e0.elapsed_time(e1) * 1e3 / 20, 2),
            'request_bytes': len(req),
            'note': 'request_ms = host JPEG/msgpack decode + uint8 upload + GPU '
                    'preprocessing + chunk graph + actions to host + reply '
                    'encoding; predict_action_ms = from the first device copy '
                    'to the actions on the host'}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--batch', type=int, default=1)
    ap.add_argument('--no-cpu', action='store_true',
                    help='skip the CPU oracle baseline')
    ap.add_argument('--no-table', action='store_true',
                    help='skip the per-kernel roofline table and the C2/C3 '
                    'phase times')
    ap.add_argument('--no-configs', action='store_true',
                    help='skip the other BASELINE configs (PI0 bs 8, PI0.5 '
                    'fp8 bs 1/8/32)')
    ap.add_argument('--no-serving', action='store_true',
                    help='skip the RTC and serving-request timings')
    ap.add_argument('--kernel-only', action='store_true',
                    help='run only the dominant kernel + a calibration copy '
                    '(for rocprofv3 --pmc passes)')
    ap.add_argument('--table-only', action='store_true',
                    help='run only the per-kernel table (every main kernel '
                    'of the chunk at its chunk shape) + a calibration copy '
                    '(for rocprofv3 --kernel-trace / --pmc passes)')
    ap.add_argument('--vjp-only', action='store_true',
                    help='run guidance-with-VJP chunks alone (the rocprofv3 '
                    'pass of the VJP kernel statistics)')
    ap.add_argument('--summarize-profiles', metavar='DIR',
                    help='write the profiles/*.md summaries into DIR/profiles '
                    'from the CSVs of the rocprofv3 passes under DIR (see '
                    'profile_commands)')
    args = ap.parse_args()
    if args.summarize_profiles:
        d = args.summarize_profiles
        summarize_profiles(d, os.path.join(d, 'profiles'))
        summarize_vjp_profile(d, os.path.join(d, 'profiles'))
        return
    if args.gpus != 1:
        print('bench.py: this build runs on one GPU; multi-GPU figures are '
              'not part of it (the path shards by request: each GPU serves '
              'whole requests)',
              file=sys.stderr)
        sys.exit(2)

    if args.kernel_only:
        kernel_only()
        return
    if args.table_only:
        table_only()
        return
    if args.vjp_only:
        vjp_only()
        return

    import torch

    from fluxvla_amd.config import PI0
    from fluxvla_amd.pi0_inference import PI0Inference
    from fluxvla_amd.weights import make_inputs, make_state_dict

    dev = torch.device('cuda', 0)
    cfg = PI0
    B = args.batch
    log('generating weights on the GPU')
    sd = make_state_dict(cfg, seed=0, device=dev)
    log('preparing model')
    model = PI0Inference(cfg, sd, device=dev, max_batch=max(B, 8))
    inp = make_inputs(cfg, batch=B, seed=1)
    dinp = {k: v.to(dev) for k, v in inp.items()}

    def step():
        return model.predict_action(dinp['images'], dinp['lang_tokens'],
                                    dinp['states'], dinp['img_masks'],
                                    dinp['lang_masks'], noise=dinp['noise'])

    log(f'warmup {args.warmup} (first call captures the graph)')
    for _ in range(max(args.warmup, 1)):
        out = step()
    torch.cuda.synchronize()
    log(f'timing {args.steps} chunks')
    times = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        out = step()
        e1.record()
        times.append((e0, e1))
    torch.cuda.synchronize()
    total = time.perf_counter() - t0
    per = sorted(a.elapsed_time(b) for a, b in times)
    ms = total * 1000.0 / args.steps
    log(f'{ms:.3f} ms/chunk (wall), median event {per[len(per) // 2]:.3f} ms')

    roof = time_dominant_kernel(model) if B == 1 else None
    roof_mfma = time_mfma_kernel(model) if B == 1 else None
    if roof:
        log(f"dominant kernel {roof['avg_us']} us, {roof['achieved']} GB/s; "
            f"MFMA kernel {roof_mfma['avg_us']} us, {roof_mfma['achieved']} "
            f"TFLOP/s (library {roof_mfma['library_us']} us)")

    table, phases = None, None
    if B == 1 and not args.no_table:
        log('per-kernel rooflines and C2/C3 phase times')
        table = kernel_table(model)
        phases = phase_times(model)
        for r in table:
            log(f"  {r['kernel']:56s} {r['avg_us']:9.2f} us "
                f"{r['achieved']:8.1f} {r['unit']} ({100 * r['frac']:.1f} %)")
        log(f'  {phases}')

    cpu, err = (None, None)
    if not args.no_cpu and B == 1:
        log('timing the CPU oracle (one chunk)')
        cpu, err = cpu_baseline(sd, cfg, inp, out)
        log(f"cpu {cpu['value']} ms on {cpu['cores']} threads; gpu vs cpu "
            f'max abs err {err:.3e}')

    rtc, serving = None, None
    if B == 1 and not args.no_serving:
        log('real-time chunking and a served request')
        rtc = rtc_times(model, dinp)
        serving = serving_latency(model, cfg, dinp)
        log(f'  rtc {rtc}')
        log(f'  serving {serving}')

    configs, fp8_parity = None, None
    if B == 1 and not args.no_configs:
        log('other BASELINE configs')
        configs, fp8_parity = other_configs(model, sd, dev,
                                           parity=not args.no_cpu)

    res = {
        'metric': METRIC,
        'value': round(ms, 3),
        'unit': 'ms',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms, 3),
        'higher_is_better': False,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16',
        'data': 'synthetic (uniform-noise images, random tokens/state/noise; '
                'seeded random-init bf16 weights)',
        'config': {
            'workload': f'PI0 chunk bs={B}: 3 views x 224^2 + 48 tokens '
                        '(prefix 816) -> SigLIP-So400m/14 x27 -> Gemma-2B x18 '
                        '-> 10 Euler steps of Gemma-300M expert x18, '
                        '50x32 actions, one HIP graph',
            'batch': B,
            'prefix_tokens': cfg.prefix_len,
            'suffix_tokens': cfg.suffix_len,
            'flow_steps': cfg.num_steps,
            'median_event_ms': round(per[len(per) // 2], 3),
        },
        'roofline': roof,
        'roofline_mfma': roof_mfma,
        'kernels': table,
        'phases': phases,
        'cpu_baseline': cpu,
        'parity': None if err is None else {
            'chunk_max_abs_err_vs_cpu_oracle': err, 'tolerance': 2e-2},
        'configs': configs,
        'fp8_parity': fp8_parity,
        'rtc': rtc,
        'serving': serving,
    }
    print(json.dumps(res), flush=True)


if __name__ == '__main__':
    main()
