"""Throughput of the integer Whisper encoder + greedy decoder on one MI355X.

Workload (default): Whisper-large shapes, full integer encoder + decoder,
batch 128 of seeded 30 s log-mels (128 x 3000), 445-step greedy decode after the
3-token start prompt (448-token context), random-init weights calibrated into
an integer checkpoint. One step = encoder over the batch + the whole greedy
decode; inputs are resident in HBM before the timed region.

Prints one JSON line: end-to-end audio-seconds/s as ``value``, plus encoder
audio-s/s, decoder tokens/s, two roofline objects and the CPU oracle timed on a
bounded sample on the host:

* ``roofline``: the kernel with the largest share of the step, the decoder's
  cross-attention over the cached audio K/V with its LayerNorm and query
  projection computed in the kernel (HBM-bound, ``XA_KERNEL``). Its launches inside
  the timed steps run in a replayed HIP graph, so its duration is taken right
  after the timed region from launches identical to the graph's (same kernel,
  same buffers, same stream) bracketed by HIP events on that stream.
  ``traffic`` is the HBM bytes per launch from rocprofv3 FETCH_SIZE and
  WRITE_SIZE counters, scaled by the same counters on a plain copy, as
  recorded in profiles/attn_decode_cross_b128_pmc.md.
* ``roofline_encoder_gemm``: the encoder GEMMs (int8 MFMA), HIP events around
  every encoder GEMM launch in the timed steps. ``traffic`` is the layer
  average of the same counters over the QKV, out-projection, FC1 and FC2
  launches (profiles/encoder_gemm_large_b128_pmc.md).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "encoder audio-sec/sec + decoder tokens/sec, large shapes; % int8 MFMA peak"
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, TOP/s
HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    # name: (shape, batch, decode steps, prompt seed (None = the Whisper start
    # prompt), description)
    "large": ("large", 128, 445, None, "Whisper-large shapes (d=1280, 20 heads, 32+32 layers, 128 mels), "
              "integer encoder + greedy decoder, batch 128, 445 greedy steps after a 3-token prompt "
              "(448-token context)"),
    "medium": ("medium", 64, 224, 4, "Whisper-medium shapes (d=1024, 16 heads, 24+24 layers), batch 64, "
               "224 greedy steps after 3 seeded uniform random prompt ids in [0, 51865)"),
    "small": ("small", 32, 128, None, "Whisper-small shapes (d=768, 12 heads, 12+12 layers), batch 32, "
              "128 greedy steps"),
    "base-encoder": ("base", 16, 0, None, "Whisper-base shapes (d=512, 8 heads, 6 layers), integer "
                     "encoder only, batch 16"),
    "tiny": ("tiny", 1, 32, None, "Whisper-tiny shapes (d=384, 4 heads, 4+4 layers), batch 1, 32 greedy "
             "steps"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _timed_sample(iw, ref, dims, steps_total: int, enc_blocks: int, dec_steps: int, seed: int = 99):
    """One 30 s sample through ``ref`` (an OracleWhisper): the encoder front end,
    ``enc_blocks`` encoder blocks (all when None) and ``dec_steps`` greedy
    steps after the prompt (all when None); returns (encoder s, decoder s)
    scaled to every block and every step, and the seconds actually spent."""
    mel = iw.synth.synthetic_mel(1, dims.n_mels, 2 * dims.n_audio_ctx, seed=seed)
    nb = dims.n_audio_layer if enc_blocks is None else min(enc_blocks, dims.n_audio_layer)
    t0 = time.perf_counter()
    x = ref.encoder_frontend(mel)
    t1 = time.perf_counter()
    for i in range(nb):
        x = ref._block(x, None, None, None, f"encoder.blocks.{i}", dims.n_audio_head, False)
    t2 = time.perf_counter()
    xa = ref._ln(x, "encoder.ln_post")
    t3 = time.perf_counter()
    enc = (t1 - t0) + (t2 - t1) * dims.n_audio_layer / max(nb, 1) + (t3 - t2)
    spent = t3 - t0
    dec = 0.0
    nd = steps_total if dec_steps is None else min(dec_steps, steps_total)
    if nd:
        prompt = iw.synth.prompt_tokens(1, dims.n_vocab)
        t4 = time.perf_counter()
        ref.greedy(xa, prompt, nd)
        dec = time.perf_counter() - t4
        spent += dec
        dec *= steps_total / nd
    return enc, dec, spent


def cpu_baseline(iw, dims, params, steps_total: int, threads: int, enc_blocks: int = 8,
                 dec_steps: int = 24) -> dict:
    """The reference's CPU algorithm timed on this host: the SIMD-shaped
    restatement (oracle/iw_cpu_simd.c: int8 dot-product tiles split over
    threads for the GEMM-shaped kernels, the row kernels and the classifier on
    one thread, as the reference's CPU backend runs them), bit-identical to the
    scalar oracle.

    * ``value``: the benchmark's own shapes, one 30 s sample (the reference
      decodes one utterance at a time): the encoder front end and
      ``enc_blocks`` encoder blocks scaled to all blocks, the prompt step and
      ``dec_steps`` greedy steps scaled to all steps, on ``threads`` threads.
    * ``tiny_full``: Whisper-tiny shapes (4 heads), batch 1, 32 greedy steps,
      run in full, on ``threads`` threads and on one thread."""
    from oracle.model_oracle import OracleWhisper
    from oracle.oracle import Oracle

    isa = "AVX-512 VNNI" if Oracle("simd").lib.iws_isa() == 1 else "AVX2"
    enc, dec, spent = _timed_sample(iw, OracleWhisper(dims, params, threads=threads, kind="simd"), dims,
                                    steps_total, enc_blocks, dec_steps)
    tiny = iw.SHAPES["tiny"]
    tp = iw.synth.calibrated_int_params(tiny, seed=2024)
    full = {}
    for thr in (threads, 1):
        te, td, ts = _timed_sample(iw, OracleWhisper(tiny, tp, threads=thr, kind="simd"), tiny, 32, None, None,
                                   seed=1)
        full[thr] = (te, td)
        spent += ts
    return {
        "value": round(30.0 / (enc + dec), 5), "unit": "audio-s/s", "cores": threads,
        "os_cpu_count": os.cpu_count(), "kind": "port",
        "sample": (f"SIMD-shaped CPU restatement of the reference kernels (oracle/iw_cpu_simd.c, {isa} "
                   f"int8 dot tiles, GEMM rows over {threads} OpenMP threads, row kernels and classifier "
                   f"on one thread) on one 30 s sample at the benchmark's shapes: encoder front end + "
                   f"{min(enc_blocks, dims.n_audio_layer)}/{dims.n_audio_layer} blocks scaled to all blocks, prompt "
                   f"step + {min(dec_steps, steps_total)}/{steps_total} greedy steps scaled to all steps; "
                   f"{spent:.1f} s of CPU work in total with the Whisper-tiny runs"),
        "encoder_s_per_sample": round(enc, 3), "decoder_s_per_sample": round(dec, 3),
        "tiny_full": {
            "workload": "Whisper-tiny shapes (d=384, 4 heads, 4+4 layers), batch 1, 32 greedy steps, in full",
            "threads": {str(t): {"value": round(30.0 / (e + d), 4), "unit": "audio-s/s",
                                 "encoder_s": round(e, 3), "decoder_s": round(d, 3)}
                        for t, (e, d) in full.items()}},
    }


PMC_SUMMARIES = (ROOT / "profiles" / "attn_decode_cross_b128_pmc.md",
                 ROOT / "profiles" / "encoder_gemm_large_b128_pmc.md",
                 ROOT / "profiles" / "encoder_mfma_large_b128_pmc.md",
                 ROOT / "profiles" / "large_b128_step_kernel_stats.md")
GEMM_TRAFFIC_KEY = "gemm_dtl_kernel (encoder layer average)"
# the decoder cross-attention kernel of the token step as profilers name it
# (the one that also computes the LayerNorm and query before it)
XA_KERNEL = "attn_decode_cross_lnq_kernel"
XA_KERNEL_PLAIN = "attn_decode_stream_kernel<2048, 3, 128, 4>"


def recorded(key: str, kernel: str):
    """A figure recorded in the committed profile summaries (a line
    ``<key> <kernel>: <value>``), or None."""
    for path in PMC_SUMMARIES:
        try:
            for line in path.read_text().splitlines():
                if line.startswith(f"{key} {kernel}:"):
                    return float(line.rsplit(":", 1)[1])
        except OSError:
            pass
    return None


def recorded_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed counter summaries
    (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy), or None."""
    return recorded("traffic_bytes_per_launch", kernel)


def cross_attention_probe(dec, dims, batch: int, launches: int = 20) -> float:
    """Average duration (ms) of the token step's cross-attention kernel (with
    its LayerNorm and query projection) on layer 0's cached K/V and the last
    step's residual rows, HIP events on the launch stream around each launch."""
    import torch

    if dec.fuse_cross:
        out = torch.empty_like(dec.wvf)
        launch = lambda: dec.cross_attention_lnq(0, out)
    else:  # head sizes other than 64: the plain kernel on a random query
        C = dims.n_text_state
        q = torch.randint(-127, 128, (batch, C), dtype=torch.int8, device="cuda")
        out = torch.empty((batch, C), dtype=torch.int8, device="cuda")
        launch = lambda: dec.cross_attention(0, q, out)
    launch()  # warm
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(launches)]
    for e0, e1 in ev:
        e0.record()
        launch()
        e1.record()
    torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in ev) / launches


def rowop_bandwidth(iw, rows: int, channels: int, batch: int, positions: int, reps: int = 10) -> dict:
    """HBM rate of the row / elementwise kernels at the encoder's activation
    sizes, each launched alone (HIP events around `reps` launches on the
    current stream): the LayerNorm every encoder block runs twice, and the
    op-level GeLU (FC1-sized input), residual15 and add_requant15 kernels
    (the model path fuses the last three into GEMM epilogues). Bytes are the
    algorithmic ones: every input read once, every output written once."""
    import torch

    L = iw._lib
    st = torch.cuda.current_stream().cuda_stream
    dev = "cuda"

    def timed(fn) -> float:
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    g = torch.Generator(device=dev).manual_seed(5)
    n = rows * channels
    out = {}

    def report(name, ms, nbytes):
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": nbytes,
                     "avg_launch_ms": round(ms, 4)}

    x16 = torch.randint(-16383, 16384, (rows, channels), dtype=torch.int16, device=dev, generator=g)
    gam = torch.randint(-127, 128, (channels,), dtype=torch.int8, device=dev, generator=g)
    bet = torch.randint(-4096, 4096, (channels,), dtype=torch.int32, device=dev, generator=g)
    o8 = torch.empty((rows, channels), dtype=torch.int8, device=dev)
    ms = timed(lambda: L.call("iw_layernorm32", x16.data_ptr(), gam.data_ptr(), bet.data_ptr(), 200, 10, 1 << 31,
                              5, 13, o8.data_ptr(), rows, channels, True, st))
    report("layernorm32_kernel", ms, 3 * n)
    del o8
    f = 4 * channels
    x8 = torch.randint(-127, 128, (rows, f), dtype=torch.int8, device=dev, generator=g)
    y8 = torch.empty_like(x8)
    lut = torch.randint(0, 256, (16,), dtype=torch.int32, device=dev, generator=g).to(torch.uint8)
    pm = torch.randint(1, 256, (f,), dtype=torch.int32, device=dev, generator=g).to(torch.uint8)
    ps = torch.randint(4, 12, (f,), dtype=torch.int8, device=dev, generator=g)
    ms = timed(lambda: L.call("iw_gelu", x8.data_ptr(), lut.data_ptr(), pm.data_ptr(), ps.data_ptr(), pm.data_ptr(),
                              ps.data_ptr(), y8.data_ptr(), rows * f, f, f, f, st))
    report("gelu16_kernel", ms, 2 * rows * f)
    del x8, y8
    br = torch.randint(-2 ** 30, 2 ** 30, (rows, channels), dtype=torch.int32, device=dev, generator=g)
    r16 = torch.empty_like(x16)
    ms = timed(lambda: L.call("iw_residual15", br.data_ptr(), x16.data_ptr(), 1234, r16.data_ptr(), n, st))
    report("residual15_kernel", ms, 8 * n)
    del br
    xe = torch.randint(-127, 128, (rows, channels), dtype=torch.int8, device=dev, generator=g)
    pe = torch.randint(-127, 128, (positions, channels), dtype=torch.int8, device=dev, generator=g)
    m16 = torch.full((channels,), 300, dtype=torch.int16, device=dev)
    s8 = torch.full((channels,), 6, dtype=torch.int8, device=dev)
    ms = timed(lambda: L.call("iw_add_requant15", xe.data_ptr(), pe.data_ptr(), m16.data_ptr(), s8.data_ptr(),
                              r16.data_ptr(), batch, positions, channels, channels, channels, st))
    report("add_requant15_16_kernel", ms, 3 * n + positions * channels)
    del xe, pe, r16, x16
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="large", choices=sorted(WORKLOADS))
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--decode-steps", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=None)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: there is no multi-GPU path "
              f"(--gpus {args.gpus} requested).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import __graft_entry__

    iw = __graft_entry__.load_package()
    shape, batch, dsteps, prompt_seed, desc = WORKLOADS[args.workload]
    batch = args.batch or batch
    dsteps = dsteps if args.decode_steps is None else args.decode_steps
    dims = iw.SHAPES[shape]
    if 3 + dsteps > dims.n_text_ctx:
        raise SystemExit("decode steps exceed the 448-token context")
    assert torch.cuda.is_available(), "bench.py needs a GPU"

    t0 = time.time()
    params = iw.synth.calibrated_int_params(dims, seed=0)
    log(f"[bench] synthetic checkpoint ({iw.synth.param_bytes(params) / 1e9:.2f} GB) "
        f"in {time.time() - t0:.1f} s")
    model = iw.Whisper_int.from_params(dims, params).cuda().eval()
    mel = torch.from_numpy(iw.synth.synthetic_mel(batch, dims.n_mels, 2 * dims.n_audio_ctx, seed=1)).cuda()
    prompt = torch.from_numpy(iw.synth.prompt_tokens(batch, dims.n_vocab, seed=prompt_seed)).cuda()
    enc = iw.EncoderRunner(model.encoder, batch)
    dec = iw.DecoderRunner(model.decoder, batch, dims.n_audio_ctx) if dsteps else None
    torch.cuda.synchronize()
    log(f"[bench] model on GPU, batch {batch}, {dsteps} decode steps")

    def step(timed: bool):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e2 = torch.cuda.Event(enable_timing=True)
        e0.record()
        feats = enc(mel)
        e1.record()
        toks = iw.greedy_decode(model, feats, prompt, dsteps, runner=dec) if dsteps else None
        e2.record()
        return e0, e1, e2, toks

    with torch.no_grad():
        for w in range(args.warmup):
            step(False)
            torch.cuda.synchronize()
            log(f"[bench] warmup {w + 1}/{args.warmup} done")
        enc.timer = []
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        evs = []
        for k in range(args.steps):
            evs.append(step(True))
            log(f"[bench] timed step {k + 1}/{args.steps} queued")
        torch.cuda.synchronize()
        wall = time.perf_counter() - t_start
        if dsteps:
            xa_ms = cross_attention_probe(dec, dims, batch)
            dec_fused = dec.fuse_cross
        rowops = rowop_bandwidth(iw, batch * dims.n_audio_ctx, dims.n_audio_state, batch, dims.n_audio_ctx)
    enc_ms = sum(e0.elapsed_time(e1) for e0, e1, _, _ in evs)
    dec_ms = sum(e1.elapsed_time(e2) for _, e1, e2, _ in evs)
    K = args.steps
    ms_per_step = wall * 1000.0 / K
    audio_s = 30.0 * batch
    value = audio_s * K / wall
    gemm = [(ops, s.elapsed_time(e)) for kind, ops, s, e in enc.timer if kind == "gemm"]
    attn = [(ops, s.elapsed_time(e)) for kind, ops, s, e in enc.timer if kind == "attention"]
    g_ops = sum(o for o, _ in gemm) / len(gemm)
    g_ms = sum(t for _, t in gemm) / len(gemm)
    g_tops = g_ops / (g_ms * 1e-3) / 1e12
    a_tops = (sum(o for o, _ in attn) / max(sum(t for _, t in attn), 1e-9)) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "audio-s/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded log-mel N(-0.5,0.4) clipped to [-1.5,1.5]; random-init N(0,0.02) "
                "weights calibrated to an integer checkpoint)",
        "config": {"workload": desc, "shape": shape, "global_batch": batch, "seq_len": dims.n_audio_ctx,
                   "decode_steps": dsteps, "parallelism": "none"},
        "encoder_audio_s_per_s": round(audio_s * K / (enc_ms / 1000.0), 2),
        "decoder_tokens_per_s": round(batch * dsteps * K / (dec_ms / 1000.0), 1) if dsteps else None,
        "encoder_ms_per_step": round(enc_ms / K, 3),
        "decoder_ms_per_step": round(dec_ms / K, 3),
        "encoder_attention_tops": round(a_tops, 1),
        "roofline_encoder_gemm": {
            "bound": "mfma", "kernel": "gemm_dtl_kernel (encoder QKV/out/FC1/FC2 launches)",
            "achieved": round(g_tops, 1), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
            "frac": round(g_tops / INT8_PEAK_TOPS, 4), "traffic": recorded_traffic(GEMM_TRAFFIC_KEY),
            "ops_per_launch": g_ops, "avg_launch_ms": round(g_ms, 4),
            # counters (profiles/encoder_mfma_large_b128_pmc.md): the fraction of the int8
            # MFMA pipes' cycles at work, SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x cycles)
            "mfma_busy_pmc": recorded("mfma_busy_pmc", GEMM_TRAFFIC_KEY)},
        "encoder_attention": {
            "kernel": "attn_prefill_kernel<2, false, true>", "achieved_tops": round(a_tops, 1),
            "ops": "4*B*H*T^2*D (QK^T and P.V)",
            "mfma_busy_pmc": recorded("mfma_busy_pmc", "attn_prefill_kernel"),
            "valu_busy_pmc": recorded("valu_busy_pmc", "attn_prefill_kernel")},
        "hbm_kernels": rowops,
    }
    if dsteps:
        # algorithmic bytes: K [Tk, D] and V [D, Tk] of every (b, h), the
        # residual rows (int16) and the query weight read once, and out
        H, D, Tk = dims.n_text_head, dims.n_text_state // dims.n_text_head, dims.n_audio_ctx
        C = H * D
        if dec_fused:
            xa_bytes = batch * H * 2 * Tk * D + batch * C * 2 + C * C + batch * C
        else:  # K, V, q and out
            xa_bytes = batch * H * (2 * Tk * D + 2 * D)
        xa_gbs = xa_bytes / (xa_ms * 1e-3) / 1e9
        kname = XA_KERNEL if dec_fused else XA_KERNEL_PLAIN
        result["roofline"] = {
            "bound": "hbm", "kernel": kname + " (decoder cross-attention"
                     + (" with its LayerNorm and query projection" if dec_fused else "")
                     + f", 1 query x {Tk} cached keys per (batch, head))",
            "achieved": round(xa_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(xa_gbs / HBM_PEAK_GBS, 4), "traffic": recorded_traffic(kname),
            "bytes_per_launch": xa_bytes, "avg_launch_ms": round(xa_ms, 4),
            "launches_per_step": dsteps * dims.n_text_layer}
        # the same kernel's average inside the replayed decode graphs, from the
        # committed kernel trace (profiles/large_b128_step_kernel_stats.md)
        tr_us = recorded("in_step_avg_us", kname)
        if tr_us and shape == "large" and batch == 128:
            result["roofline"]["avg_launch_ms_in_step_trace"] = round(tr_us / 1000.0, 5)
            result["roofline"]["frac_in_step_trace"] = round(xa_bytes / (tr_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    del model, enc, dec
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(os.cpu_count() or 1, 16)
        t0 = time.time()
        result["cpu_baseline"] = cpu_baseline(iw, dims, params, dsteps, threads)
        log(f"[bench] cpu baseline in {time.time() - t0:.1f} s")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
