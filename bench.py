"""Benchmark of the Sana-0.6B DiT forward on one MI355X.

Workload: the full 28-block forward at 1024 px (latent 32x32x32, 1024 image
tokens), CFG batch 2 (the latent is read twice), 300 caption tokens of width
2304 projected on the GPU, timestep 999, self-attention 36x32 heads and
cross-attention 16x72 heads, seeded N(0, 0.02) weights, all on one GPU.

A timed step is one sana_dit_step_device call: caption projection, the
cross-attention K/V of all 28 blocks and the DiT forward (patch embed, time
MLP, 28 blocks, final layer) -> velocity [2, 32, 32, 32].  That is strictly
more work than the reference's per-step forward, which reuses the projected
caption across steps (src/transformer.cpp:701-708).  The per-step cost with
the context kept resident (sana_dit_forward_device) is reported beside it.

Prints ONE JSON line (rank 0, N = 1 only):
  value / ms_per_step      ms per step (lower is better)
  kernels                  every kernel class of a block, timed with HIP events
                           on the stream it runs on, launched exactly as the
                           forward launches it (sana_dit_time_kernel: same
                           instantiation and per-CFG-branch shape, weights
                           cycled over the 28 blocks), with its algorithmic
                           flops / bytes, the bound, the achieved rate against
                           the MI355X peak and the HBM bytes per launch from the
                           rocprofv3 FETCH_SIZE / WRITE_SIZE summary in profiles/
  roofline                 the forward's dominant kernel (largest total time
                           per forward; roles that share one kernel
                           instantiation are one kernel, as in a trace)
  cpu_baseline             the reference's own CPU code (compiled from source
                           into oracle/_ref, 1 thread, CPU model named) on the
                           same seeded weights and inputs: one full CFG step at
                           this workload (caption projection + 28-block
                           forward); beside it the single-block configuration
                           (B=1, 256 tokens, 16x72 heads, median of 3), the
                           4096-token linear attention + Mix-FFN
                           microbenchmark (median of 3), the 20-step loop
                           (extrapolated from the step) and the 4096 px forward
                           (extrapolated from one 16384-token block)
  peaks_measured           the dense fp16 MFMA rate of independent MFMA
                           accumulators (sana_hip_mfma_peak, one workgroup per
                           CU) and the HBM rate of 4 GiB streaming reads and
                           copies (sana_hip_hbm_peak), on this GPU
  forward_roofline         lower bound of the step, sum over kernels of
                           max(flops / MFMA peak, bytes / HBM peak), with the
                           spec (headline) and the measured peaks, and the
                           measured step as a fraction of it

  forward_4096px           the same forward at latent 128x128 (16384 tokens,
                           CFG batch 2), context resident
  kernels_4096px           the kernel table at 16384 tokens per branch, where
                           the working sets exceed the 256 MB last-level cache
  microbench_4096_tokens   linear attention and Mix-FFN at 4096 tokens
  vae_decode_1024px        the DC-AE decode of one 32x32x32 latent to a
                           1024x1024 image (the stage after the denoising
                           loop), ms and TFLOP/s
  gemma_encode_prompt_pair the Gemma-2 2B text encoder over the prompt
                           pair's two sequences (the stage before the loop),
                           ms and TFLOP/s
  model_load_gguf          seconds to load the 28-block model from a GGUF
                           file (F32 and F16 payloads) into a fresh context

--pmc-calib adds, before the timed region, three launches of a plain copy
kernel over 256 MiB (torch.neg: 256 MiB read + 256 MiB written), the known
size the HBM counters are scaled by.
"""
import argparse
import json
import os
import re
import shutil
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sana.cpp_amd"))

PEAK_MFMA_TFLOPS = 2516.6   # MI355X dense fp16/bf16
PEAK_HBM_GBS = 8000.0

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "dit_kernels_1024px_hbm_traffic.md")
TRAFFIC_FILE_4096 = os.path.join(ROOT, "profiles", "dit_kernels_4096px_hbm_traffic.md")
CPU_REPS = 3

DIMS = dict(layers=28, hidden=1152, ffn=5760, caption_dim=2304, latent_channels=32, self_heads=36, cross_heads=16)
SIDE = 32          # 1024 px / 32 (DC-AE f32 latent)
CAPTION_LEN = 300
TIMESTEP = 999.0


def forward_flops(B, N, L, d=DIMS, with_context=True):
    """Dense-contraction FLOPs of one forward (2 per multiply-add)."""
    C, E, F, Cl = d["hidden"], d["ffn"], d["ffn"] // 2, d["latent_channels"]
    Hs, Hc = d["self_heads"], d["cross_heads"]
    Ds, Dc = C // Hs, C // Hc
    M = B * N
    blk = (2 * M * C * 3 * C                         # fused q|k|v
           + 2 * 2 * B * N * Hs * (Ds + 1) * Ds     # K^T[V|1] state + Q.[S|ksum]
           + 3 * 2 * M * C * C                       # attn out, cross q, cross out
           + 2 * 2 * B * Hc * N * L * Dc             # Q.K^T and P.V
           + 2 * M * C * E + 2 * M * E * 9 + 2 * M * F * C)  # inverted, depthwise, point
    ctx_kv = 2 * 2 * B * L * C * C                   # cross K and V of one block
    total = d["layers"] * (blk + (ctx_kv if with_context else 0))
    total += 2 * M * Cl * C + 2 * M * C * Cl          # patch embed, proj_out
    total += 2 * B * (256 * C + C * C + C * 6 * C)    # time MLP
    if with_context:
        total += 2 * B * L * d["caption_dim"] * C + 2 * B * L * C * C   # caption projection
    return total


def step_lower_bound_ms(B, N, L, p_mfma_tflops, p_hbm_gbs, d=DIMS):
    """Roofline lower bound of one step: every kernel at max(flops / MFMA peak,
    bytes / HBM peak).  GEMMs are counted by flops; the bandwidth kernels by
    their compulsory fp16 activation / fp32 residual interface bytes (no
    re-reads, no weights): LN+modulate x2, linear attention, cross attention,
    dwconv+GLU."""
    C, E, F = d["hidden"], d["ffn"], d["ffn"] // 2
    Hs, Hc = d["self_heads"], d["cross_heads"]
    Ds, Dc = C // Hs, C // Hc
    M = B * N
    fl = lambda f: f / (p_mfma_tflops * 1e12) * 1e3
    by = lambda b: b / (p_hbm_gbs * 1e9) * 1e3
    gemm = 2 * M * C * 3 * C + 3 * 2 * M * C * C + 2 * M * C * E + 2 * M * F * C + 2 * 2 * B * L * C * C
    blk = fl(gemm)
    blk += 2 * by(M * C * 4 + M * C * 2)                                       # LN + modulate
    blk += max(fl(2 * 2 * B * N * Hs * (Ds + 1) * Ds), by(4 * M * C * 2))     # linear attention
    blk += max(fl(2 * 2 * B * Hc * N * L * Dc), by(2 * M * C * 2 + 2 * B * L * C * 2))   # cross attention
    blk += max(fl(2 * M * E * 9), by(M * E * 2 + M * F * 2))                  # dwconv + GLU
    total = d["layers"] * blk
    total += fl(2 * M * d["latent_channels"] * C * 2 + 2 * B * (256 * C + C * C + C * 6 * C))
    total += fl(2 * B * L * d["caption_dim"] * C + 2 * B * L * C * C)
    return total


def measured_peaks(sana_dit, torch, dev, stream):
    """MFMA ceilings from sana_hip_mfma_peak (1024 workgroups of 4 waves, 8
    independent accumulators per wave; fp16 operands spread over [-1, 1), and
    all zero) and HBM rates from sana_hip_hbm_peak over 4 GiB (read only, and
    copy), timed with HIP events on `stream`."""
    import ctypes
    L = sana_dit.lib()
    sp = stream.cuda_stream
    wg, iters = 1024, 2000
    sink = torch.empty(wg * 256, device=dev, dtype=torch.float32)
    fl = ctypes.c_double()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    mfma = {}
    for zero in (0, 1):
        sana_dit.check(L.sana_hip_mfma_peak(wg, iters, zero, sink.data_ptr(), sp, ctypes.byref(fl)))
        e0.record(stream)
        for _ in range(3):
            sana_dit.check(L.sana_hip_mfma_peak(wg, iters, zero, sink.data_ptr(), sp, ctypes.byref(fl)))
        e1.record(stream)
        torch.cuda.synchronize()
        mfma[zero] = fl.value * 3 / (e0.elapsed_time(e1) * 1e-3) / 1e12
    nbytes = 4 << 30
    nsink = ctypes.c_int64()
    sana_dit.check(L.sana_hip_hbm_peak(None, None, 0, None, ctypes.byref(nsink), None))
    hsink = torch.empty(nsink.value, device=dev, dtype=torch.float32)
    src = torch.ones(nbytes // 4, device=dev, dtype=torch.float32)
    dst = torch.empty_like(src)
    rates = {}
    for mode in ("read", "copy"):
        def once():
            sana_dit.check(L.sana_hip_hbm_peak(src.data_ptr(), dst.data_ptr() if mode == "copy" else None, nbytes,
                                               hsink.data_ptr(), None, sp))
        once()
        e0.record(stream)
        for _ in range(4):
            once()
        e1.record(stream)
        torch.cuda.synchronize()
        moved = nbytes * (2 if mode == "copy" else 1)
        rates[mode] = 4 * moved / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst, sink, hsink
    return {"mfma_tflops": round(mfma[0], 1), "mfma_tflops_zero_operands": round(mfma[1], 1),
            "hbm_read_gbs": round(rates["read"], 1), "hbm_copy_gbs": round(rates["copy"], 1),
            "hbm_gbs": round(max(rates.values()), 1),
            "how": "MFMA: 1024 workgroups x 4 waves, 8 independent fp16 32x32x16 accumulators per wave, no memory "
                   "traffic, operands spread over [-1, 1) (mfma_tflops, the rate random weights see) and all zero "
                   "(power-limited part: zeros run faster); HBM: 16-byte grid-stride streaming over 4 GiB, read only "
                   "and copy (read + write)"}


def progress(msg):
    """One line per finished phase on stderr (stdout carries only the JSON line)."""
    print(f"bench.py: {msg}", file=sys.stderr, flush=True)


def _harness(*args, timeout=600):
    exe = os.path.join(ROOT, "oracle", "_ref", "ref_harness")
    cmd = [exe] + [str(a) for a in args]
    if shutil.which("taskset"):
        cmd = ["taskset", "-c", "0"] + cmd
    t0 = time.time()
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if out.returncode != 0:
        raise RuntimeError("reference CPU baseline failed: " + out.stderr[-500:])
    progress(f"cpu baseline: ref_harness {' '.join(str(a) for a in args)} done in {time.time() - t0:.1f} s")
    vals = {}
    for ln in out.stdout.splitlines():
        parts = ln.split()
        if len(parts) == 2:
            try:
                vals[parts[0]] = float(parts[1])
            except ValueError:
                pass
    return vals


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or the platform string."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def cpu_baseline(quick=False):
    """The reference's own CPU code (oracle/_ref/ref_harness, built from the
    reference's sources), 1 thread pinned to core 0, on the same seeded weights
    (0.02 * randn_torch_cpu(shape, 1000 + sorted index)) and inputs (latent
    seed 42, caption seed 43) as the GPU leg: one full CFG step of this
    workload (caption projection + 28-block forward), plus the single-block
    configuration, the 4096-token microbenchmark and one block at 16384
    tokens; the 20-step loop and the 4096 px forward are extrapolated from
    them.  quick: one block x 28 instead of the full step."""
    exe = os.path.join(ROOT, "oracle", "_ref", "ref_harness")
    if not os.path.exists(exe):
        return None
    t0 = time.time()
    res = {"unit": "ms/step", "cores": 1, "kind": "reference", "host_nproc": os.cpu_count(),
           "cpu_model": cpu_model()}
    if quick:
        blk = _harness("time-block", DIMS["self_heads"], DIMS["cross_heads"], 2, SIDE, CPU_REPS)["median_block_ms"]
        res["value"] = round(blk * DIMS["layers"], 1)
        res["sample"] = (f"extrapolated: one reference block_forward at B=2, N=1024, L=300, 36x32/16x72 heads, "
                         f"median of {CPU_REPS} ({blk:.0f} ms), x28 blocks")
        fwd_ms, cap_ms = res["value"], 0.0
    else:
        v = _harness("time-forward", DIMS["self_heads"], DIMS["cross_heads"], SIDE, timeout=900)
        res["value"] = round(v["step_ms"], 1)
        res["forward_ms"] = round(v["forward_ms"], 1)
        res["caption_projection_ms"] = round(v["caption_projection_ms"], 1)
        res["sample"] = ("one full CFG step as the reference runs it: caption projection (300x2304 -> 1152) + "
                         "the 28-block forward of run_full_denoising_step_with_cfg at 1024 px, batch 2, t=999, "
                         "36x32/16x72 heads, seeded N(0,0.02) weights, 1 thread")
        fwd_ms, cap_ms = v["forward_ms"], v["caption_projection_ms"]
    # the 20-step loop at 1024 px: the reference's loop projects the caption
    # once and runs 20 CFG forwards (src/transformer.cpp:692-724); the solver
    # update is negligible
    res["loop_20_steps_1024px_ms"] = round(20 * fwd_ms + cap_ms, 1)
    res["loop_20_steps_note"] = "extrapolated: 20 x the forward above + one caption projection"
    # the 4096 px forward: one block at 16384 tokens (B=1), x 2 batch rows x 28 blocks
    b16k = _harness("time-block", DIMS["self_heads"], DIMS["cross_heads"], 1, 128, 1, timeout=900)
    res["block_16384_tokens_ms"] = round(b16k["median_block_ms"], 1)
    res["forward_4096px_ms"] = round(b16k["median_block_ms"] * 2 * DIMS["layers"], 1)
    res["forward_4096px_note"] = ("extrapolated: one reference block_forward at B=1, 128x128 latent (16384 tokens), "
                                  "36x32/16x72 heads, L=300 (1 run), x 2 CFG batch rows x 28 blocks; the caption "
                                  "projection is left out (context resident, as the GPU forward_4096px line)")
    b256 = _harness("time-block", 16, 16, 1, 16, CPU_REPS)
    res["block_256_tokens_ms"] = round(b256["median_block_ms"], 1)
    micro = _harness("time-micro", 64, CPU_REPS, timeout=900)
    res["linear_attention_4096_tokens_ms"] = round(micro["median_linear_attention_ms"], 1)
    res["mixffn_4096_tokens_ms"] = round(micro["median_mixffn_ms"], 1)
    res["block_and_micro_note"] = ("block_256_tokens: one block_forward, B=1, 16x16 latent (256 tokens), 16x72 self "
                                   f"heads as written, L=300, median of {CPU_REPS}; linear_attention / mixffn "
                                   "4096 tokens: linear_attention_4d on [2,16,4096,72] and glumb_conv on "
                                   f"[2,1152,64,64], median of {CPU_REPS}")
    res["wall_s"] = round(time.time() - t0, 1)
    return res


def model_load_times(sana_dit, torch, weights):
    """GGUF -> device load of the 28-block model through sana_dit_load_gguf: one
    file holding every tensor (model, caption and denoiser names), written as
    F32 (the reference's payload type) and as F16 (the linear weights go to the
    fp16 operand buffers as stored, no fp32 round trip), each into a fresh
    context.  The file was just written, so it is read from the page cache:
    this is the host-side conversion + upload cost, not disk speed.  Then the
    same F32 file through sana_dit_load_gguf_cached: the first call loads the
    GGUF and writes the packed device-layout cache, the second loads the cache
    (both into fresh contexts)."""
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from gguf_writer import GGML_F16, GGML_F32, write_gguf
    out = {}
    tmp = tempfile.mkdtemp(prefix="sana_bench_")
    try:
        for tag, ty in (("f32", GGML_F32), ("f16", GGML_F16)):
            path = os.path.join(tmp, f"model_{tag}.gguf")
            write_gguf(path, weights, ggml_type=ty)
            size = os.path.getsize(path)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            d = sana_dit.Dit(**DIMS, device=0)
            d.load_gguf(path, path, path)
            d.check_weights()
            torch.cuda.synchronize()
            sec = time.perf_counter() - t0
            d.close()
            out[tag] = {"s": round(sec, 3), "file_gb": round(size / 1e9, 3), "gb_per_s": round(size / 1e9 / sec, 2)}
            progress(f"GGUF load ({tag}) {sec:.2f} s")
            if tag == "f32":
                cache = os.path.join(tmp, "model.sanapk")
                for key in ("f32_cache_write", "packed_cache"):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    d = sana_dit.Dit(**DIMS, device=0)
                    used = d.load_gguf_cached(path, path, path, cache)
                    d.check_weights()
                    torch.cuda.synchronize()
                    sec = time.perf_counter() - t0
                    d.close()
                    if used != (key == "packed_cache"):
                        raise RuntimeError(f"packed cache {'not ' if used is False else ''}used in {key}")
                    out[key] = {"s": round(sec, 3), "file_gb": round(os.path.getsize(cache) / 1e9, 3)}
                    progress(f"GGUF load through the packed cache ({key}) {sec:.2f} s")
                os.remove(cache)
            os.remove(path)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    out["note"] = ("sana_dit_load_gguf of the 28 blocks + caption + denoiser tensors from one GGUF file in the page "
                   "cache into a fresh context (context creation included); f32_cache_write: the same F32 file "
                   "through sana_dit_load_gguf_cached with no cache (GGUF load + packed image written); "
                   "packed_cache: the second such call, from the packed device-layout image")
    return out


def microbench_4096(sana_dit, torch, dev, stream):
    """Linear attention (16 heads x 72) and the Mix-FFN (inverted GEMM + SiLU,
    depthwise 3x3 + GLU, point GEMM + gated residual) at 64x64 = 4096 tokens,
    batch 2, through the kernel-level launchers on `stream`."""
    L = sana_dit.lib()
    B, N, H, D, C, E = 2, 4096, 16, 72, 1152, 5760
    F, M = E // 2, 2 * 4096
    g = torch.Generator(device=dev).manual_seed(5)
    q, k, v = (torch.randn((M, C), device=dev, dtype=torch.float16, generator=g) for _ in range(3))
    o = torch.empty((M, C), device=dev, dtype=torch.float16)
    ws = torch.empty(L.sana_hip_linear_attention_workspace(B, N, H, D) // 4 + 1, device=dev, dtype=torch.float32)
    x16 = torch.randn((M, C), device=dev, dtype=torch.float16, generator=g)
    w_inv = torch.randn((E, C), device=dev, dtype=torch.float16, generator=g) * 0.02
    b_inv = torch.zeros(E, device=dev)
    hid = torch.empty((M, E), device=dev, dtype=torch.float16)
    w_dw = torch.randn((9, E), device=dev, generator=g) * 0.2
    b_dw = torch.zeros(E, device=dev)
    glu = torch.empty((M, F), device=dev, dtype=torch.float16)
    w_pt = torch.randn((C, F), device=dev, dtype=torch.float16, generator=g) * 0.02
    x32 = torch.zeros((M, C), device=dev)
    sp = stream.cuda_stream
    torch.cuda.synchronize()

    def la():
        sana_dit.check(L.sana_hip_linear_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), C, o.data_ptr(), C, B, N,
                                                   H, D, ws.data_ptr(), sp))

    def ffn_parts():
        sana_dit.check(L.sana_hip_gemm(x16.data_ptr(), C, w_inv.data_ptr(), C, M, E, C, b_inv.data_ptr(), 1,
                                       hid.data_ptr(), E, None, 0, sp))
        sana_dit.check(L.sana_hip_dwconv_glu(hid.data_ptr(), E, w_dw.data_ptr(), b_dw.data_ptr(), glu.data_ptr(), F, B,
                                             64, 64, F, sp))
        sana_dit.check(L.sana_hip_gemm_residual(glu.data_ptr(), F, w_pt.data_ptr(), F, M, C, F, None, None, None, 0, N,
                                                x32.data_ptr(), C, None, 0, sp))

    def timed(fn, it=20):
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(it):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / it * 1e3

    la_us = timed(la)
    ffn_us = timed(ffn_parts)
    la_bytes = 4 * M * C * 2                      # q, k, v in, out
    ffn_flops = 2 * M * E * C + 2 * M * C * F
    return {"linear_attention_us": round(la_us, 2), "linear_attention_GBs": round(la_bytes / (la_us * 1e-6) / 1e9, 1),
            "mixffn_us": round(ffn_us, 2), "mixffn_tflops": round(ffn_flops / (ffn_us * 1e-6) / 1e12, 1),
            "shape": "B=2, 64x64 tokens, C=1152, self heads 16x72, Mix-FFN 1152->5760->2880->1152"}


VAE_CHANNELS = (128, 256, 512, 512, 1024, 1024)   # DC-AE f32c32 decoder of Sana 1.0, level 0 = output
VAE_ATTENTION = (False, False, False, True, True, True)


def vae_flops(h, w, channels=VAE_CHANNELS, attention=VAE_ATTENTION, latent=32, head=32, expand=4):
    """Multiply-add flops (x2) of one DC-AE decode of an h x w latent: 3x3 convs
    as 9-tap GEMMs, the multiscale attention (q|k|v, depthwise 5x5, grouped
    1x1, two linear attentions, to_out) and GLUMBConv."""
    L = len(channels)
    f = 2 * 9 * latent * channels[-1] * h * w
    for i in range(L - 1, -1, -1):
        C, s = channels[i], 2 ** (L - 1 - i)
        P = h * s * w * s
        if i + 1 < L:
            f += 2 * 9 * channels[i + 1] * C * P
        for _ in range(3):
            if not attention[i]:
                f += 2 * (2 * 9 * C * C * P)
            else:
                E = expand * C
                f += 2 * P * 3 * C * C + 2 * 25 * 3 * C * P + 2 * head * 3 * C * P
                f += 2 * (C // head) * 2 * (2 * (head + 1) * head * P)
                f += 2 * P * C * 2 * C + 2 * P * 2 * E * C + 2 * 9 * 2 * E * P + 2 * P * C * E
    return f + 2 * 9 * channels[0] * 3 * h * w * 4 ** (L - 1)


def vae_decode_1024px(sana_dit, torch, dev, stream, rng):
    """DC-AE decode of one 32x32x32 latent to a 1024x1024 image on the device
    (sana_vae_decode_device), seeded N(0, 0.02) weights, RMSNorm weights
    1 + 0.1 N(0, 1); mean of 3 decodes after one warm-up."""
    import numpy as np
    v = sana_dit.Vae(VAE_CHANNELS, VAE_ATTENTION)
    for name, shape in sana_dit.vae_manifest(VAE_CHANNELS, VAE_ATTENTION).items():
        z = rng.standard_normal(shape, dtype=np.float32)
        norm = name.endswith("norm.weight") or name.endswith("norm_out.weight")
        v.set_weight(name, 1 + np.float32(0.1) * z if norm else z * np.float32(0.02))
    v.check_weights()
    lat = torch.from_numpy(rng.standard_normal((1, 32, SIDE, SIDE), dtype=np.float32)).to(dev)
    img = torch.empty((1, 3, 1024, 1024), device=dev, dtype=torch.float32)
    sp = stream.cuda_stream
    v.decode_device(lat, tuple(lat.shape), img, sp)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(3):
        v.decode_device(lat, tuple(lat.shape), img, sp)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 3
    if not torch.isfinite(img).all():
        raise RuntimeError("non-finite decoded image")
    v.close()
    fl = vae_flops(SIDE, SIDE)
    return {"ms": round(ms, 3), "tflops": round(fl / (ms * 1e-3) / 1e12, 1), "gflop": round(fl / 1e9, 1),
            "shape": "latent 1x32x32x32 -> image 1x3x1024x1024, DC-AE f32c32 (128/256/512 ResBlocks, "
                     "512/1024/1024 EfficientViT)"}


def gemma_flops(T, c):
    """2 x multiply-adds of one Gemma-2 encoder pass over T tokens: the q|k|v,
    output, gate|up and down projections, and the causal score and P.V
    products (full T x T, as computed)."""
    H, Dq, Dkv, F = c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"], c["ffn"]
    per_layer = 2 * T * (H * (Dq + 2 * Dkv) + Dq * H + 3 * H * F) + 2 * 2 * T * T * Dq
    return c["layers"] * per_layer


def gemma_prompt_pair(sana_dit, rng, pos_tokens=438, neg_tokens=300):
    """Gemma-2 2B encoder (26 layers, 256000-token vocabulary) on the two
    sequences encode_prompt_pair runs: the instruction-prefixed positive
    prompt (instruction + 300 - 2 tokens) and the negative prompt (300).
    Seeded N(0, 0.02) weights, one draw per tensor shape shared by the 26
    layers; both sequences in one pass (sana_gemma_encode_pair, as the host
    encode_prompt_pair runs them); mean of 3 pairs after one warm-up."""
    import numpy as np
    c = sana_dit.GEMMA2_2B
    g = sana_dit.Gemma(c)
    by_shape = {}
    for name, shape in sana_dit.gemma_manifest(**c).items():
        if shape not in by_shape:
            z = rng.standard_normal(shape, dtype=np.float32)
            by_shape[shape] = 1 + np.float32(0.1) * z if len(shape) == 1 else z * np.float32(0.02)
        g.set_weight(name, by_shape[shape])
    g.check_weights()
    pos = rng.integers(0, c["vocab"], size=pos_tokens)
    neg = rng.integers(0, c["vocab"], size=neg_tokens)
    g.encode_pair(pos, neg)
    t0 = time.perf_counter()
    for _ in range(3):
        h, _ = g.encode_pair(pos, neg)
    ms = (time.perf_counter() - t0) * 1e3 / 3
    if not np.isfinite(h).all():
        raise RuntimeError("non-finite Gemma hidden states")
    g.close()
    fl = gemma_flops(pos_tokens, c) + gemma_flops(neg_tokens, c)
    return {"ms": round(ms, 3), "tflops": round(fl / (ms * 1e-3) / 1e12, 1), "gflop": round(fl / 1e9, 1),
            "shape": f"Gemma-2 2B, {pos_tokens} + {neg_tokens} tokens, host token ids in, host hidden states out"}


def measured_traffic(path=TRAFFIC_FILE):
    """Bytes per launch of each kernel role (qkv, attn_out, ...) from a
    committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary of the same kernel
    table ({role: bytes}; empty when absent)."""
    try:
        text = open(path).read()
    except OSError:
        return {}
    return {m.group(1): int(m.group(2))
            for m in re.finditer(r"^traffic_bytes_per_launch\s+(.+?):\s*([0-9]+)\s*$", text, re.M)}


KERNEL_BOUND = {"qkv": "mfma", "attn_out": "mfma", "cross_q": "mfma", "cross_out": "mfma", "ffn_inverted": "mfma",
                "ffn_point": "mfma", "ln_modulate": "hbm", "linear_attention": "hbm", "cross_attention": "hbm",
                "dwconv_glu": "hbm"}
LAUNCHES_PER_BLOCK = {"ln_modulate": 2}   # per batch-row chain; every other class runs once


def kernel_table(d, branches, traffic):
    """Every block kernel at its in-forward launch (sana_dit_time_kernel)."""
    out = {}
    chains = 2 if branches else 1
    for which, cls in enumerate(d.KERNELS):
        ms, fl, by, name = d.time_kernel(which, 2 * DIMS["layers"])
        bound = KERNEL_BOUND[cls]
        us = ms * 1e3
        if bound == "mfma":
            achieved, peak, unit = fl / (us * 1e-6) / 1e12, PEAK_MFMA_TFLOPS, "TFLOP/s"
        else:
            achieved, peak, unit = by / (us * 1e-6) / 1e9, PEAK_HBM_GBS, "GB/s"
        out[cls] = {"kernel": name, "avg_us": round(us, 2),
                    "launches_per_forward": DIMS["layers"] * chains * LAUNCHES_PER_BLOCK.get(cls, 1),
                    "gflop": round(fl / 1e9, 4), "mbytes": round(by / 1e6, 3), "bound": bound,
                    "achieved": round(achieved, 1), "peak": peak, "unit": unit, "frac": round(achieved / peak, 4),
                    "traffic": traffic.get(cls)}
    return out


def dominant_roofline(kernels):
    """The kernel (instantiation) with the largest total time per forward; the
    roles that launch the same instantiation are one kernel, as in a trace."""
    groups = {}
    for cls, k in kernels.items():
        g = groups.setdefault(k["kernel"], {"roles": [], "time": 0.0, "launches": 0, "flops": 0.0, "bytes": 0.0,
                                             "bound": k["bound"], "traffic": 0.0})
        n = k["launches_per_forward"]
        g["roles"].append(cls)
        # measured bytes per launch, averaged over the roles' launches like `bytes`
        g["traffic"] = None if g["traffic"] is None or k["traffic"] is None else g["traffic"] + k["traffic"] * n
        g["time"] += k["avg_us"] * n
        g["launches"] += n
        g["flops"] += k["gflop"] * 1e9 * n
        g["bytes"] += k["mbytes"] * 1e6 * n
    name, g = max(groups.items(), key=lambda kv: kv[1]["time"])
    avg_us = g["time"] / g["launches"]
    if g["bound"] == "mfma":
        achieved, peak, unit = g["flops"] / (g["time"] * 1e-6) / 1e12, PEAK_MFMA_TFLOPS, "TFLOP/s"
    else:
        achieved, peak, unit = g["bytes"] / (g["time"] * 1e-6) / 1e9, PEAK_HBM_GBS, "GB/s"
    return {"bound": g["bound"], "kernel": name, "roles": g["roles"], "achieved": round(achieved, 1), "peak": peak,
            "unit": unit, "frac": round(achieved / peak, 4),
            "traffic": None if g["traffic"] is None else round(g["traffic"] / g["launches"]),
            "algorithmic_bytes": round(g["bytes"] / g["launches"]), "avg_us": round(avg_us, 2),
            "launches_per_forward": g["launches"], "share_of_kernel_time": None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-quick", action="store_true",
                    help="CPU baseline from one reference block x 28 instead of the full reference step")
    ap.add_argument("--pmc-calib", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the extra 4096 px forward and 4096-token microbenchmark lines (profiling runs)")
    ap.add_argument("--extras-4096px-only", action="store_true",
                    help="of the extras, run only the 4096 px forward and its kernel table (profiling runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU (asked for {args.gpus}); "
              "the multi-GPU sharding of the path is a design only", file=sys.stderr)
        sys.exit(2)

    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_quick)   # before the GPU is touched

    import numpy as np
    import torch
    import sana_dit

    if not torch.cuda.is_available():
        raise RuntimeError("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    d = sana_dit.Dit(**DIMS, device=0)
    rng = np.random.default_rng(1234)
    # the reference CPU baseline's seeded weights and inputs (torch.randn CPU generator)
    weights = dict(sana_dit.seeded_weights(DIMS["layers"], DIMS["hidden"], DIMS["ffn"], DIMS["caption_dim"],
                                           DIMS["latent_channels"]))
    for name, w in weights.items():
        d.set_weight(name, w)
    d.check_weights()
    progress("seeded weights uploaded")

    B, N, L = 2, SIDE * SIDE, CAPTION_LEN
    latent = torch.from_numpy(sana_dit.randn((1, DIMS["latent_channels"], SIDE, SIDE), 42)).to(dev)
    caption = torch.from_numpy(sana_dit.randn((B, L, DIMS["caption_dim"]), 43)).to(dev)
    out = torch.empty((B, DIMS["latent_channels"], SIDE, SIDE), device=dev, dtype=torch.float32)
    stream = torch.cuda.Stream(device=dev)      # default priority; every launch and event below uses it
    sp = stream.cuda_stream
    shape = tuple(latent.shape)

    def step():
        d.step_device(caption, L, None, latent, shape, TIMESTEP, out, sp)

    def fwd():
        d.forward_device(latent, shape, TIMESTEP, out, sp)

    if args.pmc_calib:
        src = torch.ones(64 << 20, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        with torch.cuda.stream(stream):
            for _ in range(3):
                torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    progress(f"{args.steps} timed steps done")
    ev_ms = ev0.elapsed_time(ev1) / args.steps
    if not torch.isfinite(out).all():
        raise RuntimeError("non-finite velocity")

    # context resident (the loop-amortised per-step cost)
    for _ in range(args.warmup):
        fwd()
    torch.cuda.synchronize()
    ev0.record(stream)
    for _ in range(args.steps):
        fwd()
    ev1.record(stream)
    torch.cuda.synchronize()
    fwd_ms = ev0.elapsed_time(ev1) / args.steps

    # every kernel class at its in-forward launch (the forward just ran), HIP events on its stream
    branches = os.environ.get("SANA_DIT_CFG_BRANCHES", "1") != "0"
    kernels = kernel_table(d, branches, measured_traffic())
    progress("kernel table at 1024 px done")
    roof = dominant_roofline(kernels)
    total_kernel_us = sum(k["avg_us"] * k["launches_per_forward"] for k in kernels.values())
    roof["share_of_kernel_time"] = round(roof["avg_us"] * roof["launches_per_forward"] / total_kernel_us, 4)

    extras = {}
    if not args.no_extras:
        # 4096 px forward (latent 128x128, 16384 image tokens, same context): context resident
        lat5 = torch.from_numpy(rng.standard_normal((1, DIMS["latent_channels"], 128, 128), dtype=np.float32)).to(dev)
        out5 = torch.empty((B, DIMS["latent_channels"], 128, 128), device=dev, dtype=torch.float32)
        d.forward_device(lat5, tuple(lat5.shape), TIMESTEP, out5, sp)
        torch.cuda.synchronize()
        ev0.record(stream)
        for _ in range(3):
            d.forward_device(lat5, tuple(lat5.shape), TIMESTEP, out5, sp)
        ev1.record(stream)
        torch.cuda.synchronize()
        c5_ms = ev0.elapsed_time(ev1) / 3
        c5_flops = forward_flops(B, 128 * 128, L, with_context=False)
        extras["forward_4096px"] = {"ms": round(c5_ms, 3), "tflops": round(c5_flops / (c5_ms * 1e-3) / 1e12, 1),
                                    "tokens": 128 * 128, "note": "28 blocks, CFG batch 2, context resident"}
        # the block kernels at 16384 tokens per batch row (working sets past the 256 MB last-level cache)
        extras["kernels_4096px"] = kernel_table(d, branches, measured_traffic(TRAFFIC_FILE_4096))
        progress("4096 px forward and kernel table done")
        if not args.extras_4096px_only:
            extras["microbench_4096_tokens"] = microbench_4096(sana_dit, torch, dev, stream)
            extras["vae_decode_1024px"] = vae_decode_1024px(sana_dit, torch, dev, stream, rng)
            extras["gemma_encode_prompt_pair"] = gemma_prompt_pair(sana_dit, rng)
            try:
                extras["model_load_gguf"] = model_load_times(sana_dit, torch, weights)
            except (OSError, RuntimeError) as e:  # e.g. no room for the 2.4 GB file: report, keep the line
                extras["model_load_gguf"] = {"error": str(e)[:300]}

    peaks = measured_peaks(sana_dit, torch, dev, stream)
    progress("peaks measured")
    lb_spec = step_lower_bound_ms(B, N, L, PEAK_MFMA_TFLOPS, PEAK_HBM_GBS)
    lb_meas = step_lower_bound_ms(B, N, L, peaks["mfma_tflops"], peaks["hbm_gbs"])

    step_flops = forward_flops(B, N, L, with_context=True)
    fwd_flops = forward_flops(B, N, L, with_context=False)
    res = {
        "metric": "DiT forward ms/step @1024px CFG b=2 (1 GPU); % MFMA & HBM roofline",
        "value": round(wall_ms, 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: the reference CPU baseline's seeded weights (0.02 x torch.randn CPU generator, seed "
                "1000 + sorted tensor index; caption_norm ones) and inputs (latent seed 42, caption seed 43)",
        "config": {"workload": "Sana-0.6B DiT forward, 28 blocks, 1024px (latent 32x32x32, 1024 tokens), "
                               "CFG batch 2, 300x2304 caption projected in-step, t=999, heads 36x32 self / 16x72 cross",
                   "global_batch": B, "tokens": N, "caption_len": L},
        "ms_per_step_events": round(ev_ms, 4),
        "ms_forward_context_resident": round(fwd_ms, 4),
        "step_tflops": round(step_flops / (wall_ms * 1e-3) / 1e12, 1),
        "step_mfma_frac": round(step_flops / (wall_ms * 1e-3) / 1e12 / PEAK_MFMA_TFLOPS, 4),
        "step_gflop": round(step_flops / 1e9, 2),
        "forward_gflop_context_resident": round(fwd_flops / 1e9, 2),
        "kernels": kernels,
        "roofline": roof,
        "cpu_baseline": cpu,
        "peaks_measured": peaks,
        "forward_roofline": {"lower_bound_ms_spec_peaks": round(lb_spec, 4), "frac_spec": round(lb_spec / wall_ms, 4),
                             "lower_bound_ms_measured_peaks": round(lb_meas, 4),
                             "frac_measured": round(lb_meas / wall_ms, 4),
                             "note": "sum over kernels of max(flops/MFMA peak, bytes/HBM peak) for one step; "
                                     "frac = lower bound / measured ms_per_step; frac_spec (MI355X spec peaks "
                                     "2516.6 TFLOP/s, 8000 GB/s) is the headline"},
        **extras,
    }
    d.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
