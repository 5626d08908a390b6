"""PI0 action-chunk latency on one MI355X (BASELINE.json metric).

Workload (BASELINE config 4 at bs=1): 3 camera views of 224x224 uniform-noise
images + 48 random prompt tokens -> SigLIP-So400m/14 (27 layers) -> Gemma-2B
prefix (18 layers, 816 tokens) -> 10 Euler flow-matching steps of the
18-layer Gemma-300M action expert against the cached prefix K/V; output the
50 x 32 action chunk.  bf16 random-init weights (seeded), synthetic inputs.
One step = one whole chunk: input staging (copy_ into the static buffers)
plus one HIP graph replay.

Also reported on the same JSON line:
  roofline      the dominant kernel (prefix GeGLU GEMM, MFMA-bound) timed live
                with HIP events on the stream it runs on;
  cpu_baseline  the CPU oracle (fp32 restatement of the reference's eager
                PyTorch path) timed on this host for one chunk;
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


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE passes (counter-calibrated)."""
    import re
    path = os.path.join(ROOT, 'profiles', 'prefix_geglu_gemm_traffic.md')
    try:
        m = re.search(r'traffic_bytes_per_launch:\s*(\d+)', open(path).read())
        return int(m.group(1)) if m else None
    except OSError:
        return None


def time_dominant_kernel(model, iters=20):
    """Prefix GeGLU GEMM (M=816, K=2048, N=16384 x 2 weights, rownorm):
    the largest single kernel of the chunk.  Times `iters` back-to-back
    launches on the current stream with HIP events."""
    import torch

    from fluxvla_amd import kernels as K
    cfg = model.cfg
    b = model._bufs[1]
    L = model.llm['layers'][0]
    x = b['pre_x'].view(-1, cfg.llm_hidden)
    h = b['pre_h']
    for _ in range(3):
        K.gemm_geglu(x, L['gate_w'], L['up_w'], out=h, rownorm_eps=cfg.rms_eps)
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(
        enable_timing=True)
    e0.record(s)
    for _ in range(iters):
        K.gemm_geglu(x, L['gate_w'], L['up_w'], out=h, rownorm_eps=cfg.rms_eps)
    e1.record(s)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / iters
    M, N, Kd = x.shape[0], L['gate_w'].shape[0], x.shape[1]
    flops = 2.0 * M * N * Kd * 2
    achieved = flops / (us * 1e-6) / 1e12
    return {
        'kernel': 'gemm_tile_kernel<128,64,GEGLU> (prefix gate/up, '
                  f'M={M} N={N}x2 K={Kd})',
        'bound': 'mfma',
        'achieved': round(achieved, 2),
        'peak': PEAK_BF16_TFLOPS,
        'unit': 'TFLOP/s',
        'frac': round(achieved / PEAK_BF16_TFLOPS, 4),
        'traffic': measured_traffic(),
        'traffic_unit': 'bytes/launch (rocprofv3 FETCH_SIZE + WRITE_SIZE)',
        'avg_us': round(us, 2),
        'flops_per_launch': flops,
    }


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
    for _ in range(iters):
        K.gemm_geglu(x, wg, wu, out=h, rownorm_eps=cfg.rms_eps)
    torch.cuda.synchronize()
    src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f'kernel-only: {iters} x gemm_geglu M={M} N={N}x2 K={Kd}; '
        '3 x copy 256 MiB')


def cpu_baseline(sd_gpu, cfg, inp, gpu_out):
    """The CPU oracle for one full chunk (bounded sample: 1 chunk)."""
    import platform

    import torch

    from oracle import pi0_oracle
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    sd = {k: v.cpu() for k, v in sd_gpu.items()}
    t0 = time.perf_counter()
    ref = pi0_oracle.predict_action(sd, cfg, inp['images'],
                                    inp['lang_tokens'], inp['states'],
                                    inp['img_masks'], inp['lang_masks'],
                                    inp['noise'])
    sec = time.perf_counter() - t0
    err = (gpu_out.cpu() - ref).abs().max().item()
    return {
        'value': round(sec * 1000.0, 1),
        'unit': 'ms/chunk',
        'cores': n,
        'kind': 'port',
        'sample': '1 full PI0 bs=1 chunk (prefix + 10 steps), fp32, '
                  f'{platform.processor() or platform.machine()}',
    }, err


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--batch', type=int, default=1)
    ap.add_argument('--no-cpu', action='store_true',
                    help='skip the CPU oracle baseline')
    ap.add_argument('--kernel-only', action='store_true',
                    help='run only the dominant kernel + a calibration copy '
                    '(for rocprofv3 --pmc passes)')
    args = ap.parse_args()
    if args.gpus != 1:
        print('bench.py: this build runs on one GPU; multi-GPU figures are '
              'not part of it (the path shards by request, see DESIGN.md)',
              file=sys.stderr)
        sys.exit(2)

    if args.kernel_only:
        kernel_only()
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
    model = PI0Inference(cfg, sd, device=dev, max_batch=B)
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
    if roof:
        log(f"dominant kernel {roof['avg_us']} us, {roof['achieved']} TFLOP/s")

    cpu, err = (None, None)
    if not args.no_cpu and B == 1:
        log('timing the CPU oracle (one chunk)')
        cpu, err = cpu_baseline(sd, cfg, inp, out)
        log(f"cpu {cpu['value']} ms on {cpu['cores']} threads; gpu vs cpu "
            f'max abs err {err:.3e}')

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
        'cpu_baseline': cpu,
        'parity': None if err is None else {
            'chunk_max_abs_err_vs_cpu_oracle': err, 'tolerance': 2e-2},
    }
    print(json.dumps(res), flush=True)


if __name__ == '__main__':
    main()
