"""Benchmark: codec frames/s at batch 1 and 512 context on one MI355X.

One step = one codec frame = one code-predictor frame launch (2-token prefill + 14 decode
steps, 15 lm-heads with greedy selection, embedding combine; 5 layers) + one backbone decode
launch (28 layers at KV length 512, codec head, suppression, greedy group-0 selection), with
random-init bf16 weights of the Qwen3-TTS 0.6B talker shapes and a KV cache filled with random
bf16 values up to position 511 (each frame writes slot 511, so every frame attends to 512).

Prints one JSON line (see the repository's bench contract) with:
  value         frames/s over the timed K frames (inputs resident in HBM, no host sync inside)
  roofline      algorithmic bytes / kernel time for the dominant kernel, timed with HIP events
                on the launch stream, against MI355X's 8 TB/s
  backbone_by_context  backbone steps/s and roofline at config 0's L = 129 and config 3's L = 2048
  cpu_baseline  the CPU oracle's HF-bf16 path (eager PyTorch, bf16 weights) on this host:
                3 warm-ups, then the median of >= 10 runs; value = config 2's greedy frame loop
                (frames/s), plus backbone steps/s at L = 129 (config 0), code-predictor steps/s
                (config 1), the 512-context frame and the prefill's tokens/s
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

# Algorithmic bytes (weights + KV traffic), per the unit definitions of the decode path:
LAYER_BYTES = 15_728_640 * 2 + 4_608          # bf16 matrices + norm gains of one layer
W_BB = 28 * LAYER_BYTES + 2_048 + 3072 * 1024 * 2               # + final norm + codec head
W_CP = 5 * LAYER_BYTES + 2_048 + 2048 * 1024 * 2 + 1024 * 2     # + final norm + 1 lm-head + 1 emb row
KV_BB = 28 * 8 * 128 * 2 * 2                  # bf16 K+V bytes per attended token
KV_CP = 5 * 8 * 128 * 4 * 2                   # f32 K+V bytes per attended token
HBM_PEAK_GBS = 8000.0

# HBM bytes per launch measured with rocprofv3 PMC counters on the same workload
# (FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000 KiB, both factors from a plain 512 MiB device copy);
# the summary with the commands is profiles/qtts_decode_kernel_frame512_pmc_traffic.md.
PMC_TRAFFIC = {"cp_frame": 2_619_539_356, "backbone_step": 987_971_947}


def backbone_bytes(L: int) -> int:
    return W_BB + KV_BB * L + KV_BB


def cp_frame_bytes() -> int:
    # 15 code-predictor steps attending to L = 2..16 (the reference's unit of work)
    return sum(W_CP + KV_CP * L + KV_CP for L in range(2, 17))


def frame_bytes(L: int = 512) -> int:
    return backbone_bytes(L) + cp_frame_bytes()


def _median(xs):
    xs = sorted(xs)
    n = len(xs)
    return xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2])


def cpu_baseline(runs: int = 10, warmup: int = 3, c2_frames: int = 64) -> dict:
    """The decode path through the oracle's HF-bf16 policy (eager PyTorch, bf16 weights,
    transformers' Qwen3 op order) on the host CPU, with every host thread. Each figure takes
    `warmup` untimed runs, then the median of at least `runs` timed runs (time.perf_counter):
      backbone_steps_per_s  config 0: one backbone step at L = 129 (128 cached tokens) + codec head
      cp_steps_per_s        config 1: the 15-group code-predictor loop of one frame (2-token
                            prefill, 14 steps, 15 lm-heads, greedy); 15 / the median frame time
      value (frames/s)      config 2's greedy frame loop: frames from a 128-token prompt (the
                            prompt's K/V seeded directly; the prefill is timed separately), each
                            frame = code-predictor loop + backbone step + codec head + greedy g0 +
                            the embedding combine fed back; c2_frames frames, 1 / the median
      frame512_frames_per_s the GPU figure's frame (backbone at L = 512)
      prefill_tokens_per_s  the prompt stepped token by token (a bounded sample)."""
    import torch
    import __graft_entry__ as ge
    from oracle.qtts_oracle import DecoderOracle, TalkerWeights, rb
    pkg = ge.import_package()
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    sd = pkg.synthetic_state_dict(seed=1234)
    tw = TalkerWeights.from_state_dict(sd, 28, 5)
    bb = DecoderOracle(tw.bb_layers, tw.bb_norm, 600, "backbone", "hf_bf16")
    cp = DecoderOracle(tw.cp_layers, tw.cp_norm, 17, "cp", "hf_bf16")
    heads = [h.to(torch.bfloat16) for h in tw.cp_heads]
    embs = [e.to(torch.bfloat16) for e in tw.cp_embeddings]
    bb_emb = tw.codec_embedding.to(torch.bfloat16)
    codec_head = tw.codec_head.to(torch.bfloat16)
    g = torch.Generator().manual_seed(9)
    bb.k[:, :, :511] = torch.randn(28, 8, 511, 128, generator=g).to(torch.bfloat16)
    bb.v[:, :, :511] = torch.randn(28, 8, 511, 128, generator=g).to(torch.bfloat16)
    text = torch.randn(1024, generator=g).to(torch.bfloat16)

    def timed(fn, n):
        ts = []
        for i in range(warmup + n):
            t = time.perf_counter()
            fn(i)
            if i >= warmup:
                ts.append(time.perf_counter() - t)
        return _median(ts)

    def cp_loop(hidden, g0):
        cp.reset()
        cp.step(rb(hidden.float()).to(torch.bfloat16), pos=0)
        h, _ = cp.step(bb_emb[g0], pos=1)
        toks = []
        for gi in range(15):
            if gi:
                h, _ = cp.step(embs[gi - 1][toks[-1]], pos=gi + 1)
            toks.append(int(torch.argmax(torch.mv(heads[gi], h.to(torch.bfloat16)).float())))
        return toks

    def bb_step(x, pos):
        hb, _ = bb.step(x, pos=pos)
        return hb, int(torch.argmax(torch.mv(codec_head, hb.to(torch.bfloat16)).float()))

    x0 = torch.randn(1024, generator=g).to(torch.bfloat16)
    h0 = torch.randn(1024, generator=g)
    t_bb = timed(lambda i: bb_step(x0, 128), runs)            # config 0: L = 129
    t_cp = timed(lambda i: cp_loop(h0, 5 + i), runs)          # config 1
    t_512 = timed(lambda i: (cp_loop(h0, 5), bb_step(x0, 511)), runs)

    # config 2, greedy: the frame loop from position 128 on, the combine fed back
    state = {"h": h0, "g0": 5, "pos": 128}

    def c2_frame(i):
        toks = [state["g0"]] + cp_loop(state["h"], state["g0"])
        acc = bb_emb[toks[0]].clone()
        for gi in range(15):
            acc = acc + embs[gi][toks[gi + 1]]
        x = acc + text
        state["h"], state["g0"] = bb_step(x, state["pos"])
        state["pos"] += 1

    t_c2 = timed(c2_frame, c2_frames)

    # the prefill: the oracle's bf16 policy over a prompt from position 0, a bounded sample
    pf = DecoderOracle(tw.bb_layers, tw.bb_norm, 520, "backbone", "hf_bf16")
    xs = torch.randn(64, 1024, generator=g).to(torch.bfloat16)
    pf.step(xs[0], pos=0)
    npf, tp0 = 0, time.perf_counter()
    while npf < 63:
        pf.step(xs[npf + 1], pos=npf + 1)
        npf += 1
        if time.perf_counter() - tp0 >= 3.0:
            break
    pf_rate = npf / (time.perf_counter() - tp0)
    return {"value": round(1.0 / t_c2, 3), "unit": "frames/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(),
            "backbone_steps_per_s": round(1.0 / t_bb, 2), "cp_steps_per_s": round(15.0 / t_cp, 2),
            "frame512_frames_per_s": round(1.0 / t_512, 3), "prefill_tokens_per_s": round(pf_rate, 2),
            "protocol": f"{warmup} warm-ups, then the median of {runs} runs ({c2_frames} frames for config 2)",
            "sample": f"HF-bf16 eager PyTorch oracle on {threads} host threads: backbone step at L=129 + codec head "
                      f"(config 0); 15-group code-predictor loop (config 1); config 2's greedy frame loop from a "
                      f"128-token prompt, {c2_frames} frames; the frame at 512 context"}


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo "model name"; read from the file, no subprocess)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def prefill_flops(S: int) -> int:
    """Algorithmic flops of the MFMA prefill of S tokens: 2 per weight element per token for the
    28 layers' projections, plus the causal attention products Q K^T and P V (S (S + 1) / 2
    query-key pairs x 128 dims x 2 products x 2 flops, 16 heads), plus the codec head of the
    last token."""
    proj = 2 * 15_728_640 * 28 * S
    attn = 2 * 2 * 128 * 16 * 28 * (S * (S + 1) // 2)
    return proj + attn + 2 * 3072 * 1024


def prefill_figures(bbg, reps: int = 5) -> dict:
    """The MFMA prefill (qtts_backbone_prefill, prompt through all 28 layers + first-token
    selection) at S = 128 (config 0's prompt) and S = 2048, timed with HIP events; roofline
    against HBM (weights read once: 887 MB + the KV written) at S = 128 and against dense bf16
    MFMA (2.5 PFLOP/s) at S = 2048."""
    import torch
    out = {}
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(11)
    for S in (128, 2048):
        x = torch.randn(S, 1024, generator=g, device="cuda").to(torch.bfloat16)
        for _ in range(2):
            bbg.decoder.set_position(0)
            bbg.decoder.prefill(x, tok, -1, False)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            bbg.decoder.set_position(0)
            bbg.decoder.prefill(x, tok, -1, False)
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) / reps * 1e-3
        bytes_ = W_BB + KV_BB * S
        fl = prefill_flops(S)
        out[f"S{S}"] = {"ms": round(t * 1e3, 3), "tokens_per_s": round(S / t, 1),
                        "hbm_gbs": round(bytes_ / t / 1e9, 1), "hbm_frac": round(bytes_ / t / 1e9 / HBM_PEAK_GBS, 4),
                        "tflops": round(fl / t / 1e12, 1), "mfma_frac": round(fl / t / 1e12 / 2500.0, 4)}
    bbg.decoder.check_error()
    return out


def backbone_figure(bbg, L: int, steps: int = 30, warmup: int = 5) -> dict:
    """The backbone step (28 layers + codec head + greedy selection) at KV length L: L - 1 cached
    random bf16 entries, each launch writing slot L - 1. Timed with HIP events on the launch
    stream over `steps` launches after `warmup`; roofline = backbone_bytes(L) / time / 8 TB/s."""
    import torch
    bb = bbg.decoder
    g = torch.Generator(device="cuda").manual_seed(100 + L)
    k = torch.randn(28, 8, L - 1, 128, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(28, 8, L - 1, 128, generator=g, device="cuda").to(torch.bfloat16)
    bb.set_kv_cache(k, v)
    del k, v
    i32 = dict(dtype=torch.int32, device="cuda")
    tok, hist = torch.zeros(1, **i32), torch.zeros(1, **i32)
    x = torch.randn(1024, generator=g, device="cuda").to(torch.bfloat16)

    def step(i):
        bb.set_position(L - 1)
        bb.decode_step_select(x, tok, hist, 0, 1.0, -1, False, False, 1.0, 0, 1.0, 0, i)

    for i in range(warmup):
        step(i)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(warmup + i)
    e1.record()
    torch.cuda.synchronize()
    bb.check_error()
    t = e0.elapsed_time(e1) / steps * 1e-3
    gbs = backbone_bytes(L) / t / 1e9
    return {"L": L, "us": round(t * 1e6, 2), "steps_per_s": round(1.0 / t, 1), "algorithmic_bytes": backbone_bytes(L),
            "achieved_gbs": round(gbs, 1), "roofline_frac": round(gbs / HBM_PEAK_GBS, 4)}


def batched_frame_bytes(lengths) -> int:
    """Algorithmic bytes of one weight-shared batch frame: every weight once for all streams, each
    stream's own KV (backbone at its length, code predictor at L = 2..16)."""
    n = len(lengths)
    bb = W_BB + sum(KV_BB * L + KV_BB for L in lengths)
    cp = sum(W_CP + n * (KV_CP * L + KV_CP) for L in range(2, 17))
    return bb + cp


def batched_c4(pkg, sd, frames: int = 30) -> dict:
    """Config 4: 8 independent streams with ragged attended lengths in [128, 1024]; one frame =
    per stream one backbone step (head + greedy g0) and one code-predictor frame. Both multi-stream
    kernels are timed: the weight-shared one (the figure) and the one-stream-per-XCD one."""
    import torch
    g = torch.Generator().manual_seed(1238)
    lengths = [int(x) for x in torch.randint(128, 1025, (8,), generator=g)]
    out = {"streams": 8, "lengths": lengths, "frames": frames}
    for mode in ("shared", "per_xcd"):
        dec = pkg.BatchedTTSDecoder(sd, 8, max_seq_len=max(lengths) + 2 * frames + 8, mode=mode)
        gd = torch.Generator(device="cuda").manual_seed(7)
        for s, L in enumerate(lengths):
            k = torch.randn(28, 8, L - 1, 128, generator=gd, device="cuda").to(torch.bfloat16)
            v = torch.randn(28, 8, L - 1, 128, generator=gd, device="cuda").to(torch.bfloat16)
            dec.set_kv_cache(s, k, v)
        i32 = dict(dtype=torch.int32, device="cuda")
        g0 = torch.zeros(8, **i32)
        toks = torch.zeros(8, 16, **i32)
        comb = torch.randn(8, 1024, generator=gd, device="cuda").to(torch.bfloat16)
        text = torch.randn(8, 1024, generator=gd, device="cuda").to(torch.bfloat16)

        def frame(i):
            hidden = dec.step_select(comb, g0, -1, frame_step=i)
            dec.cp_frames(hidden, g0, text, toks, comb, frame_step=i)

        frame(0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(frames):
            frame(1 + i)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
        dec.check_error()
        if mode == "shared":
            # the streams attend lengths[s] + 1 .. + frames over the timed frames
            mid = [L + 1 + frames // 2 for L in lengths]
            nbytes = batched_frame_bytes(mid)
            gbs = nbytes * frames / el / 1e9
            out.update({"frames_per_s_total": round(8 * frames / el, 2), "frames_per_s_per_stream": round(frames / el, 2),
                        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                     "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_batch_frame": nbytes,
                                     "note": "weights counted once per batch frame (both launches), KV per stream"}})
        else:
            out["per_xcd_frames_per_s_total"] = round(8 * frames / el, 2)
        del dec
        torch.cuda.synchronize()
    out["note"] = ("weight-shared: one backbone launch and one code-predictor launch for all 8 streams per frame, "
                   "every weight read once (bf16 MFMA); per_xcd: stream s on XCD s, each XCD reading all weights")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=10, help="timed runs per CPU-baseline figure (median)")
    ap.add_argument("--backbone-context", type=int, default=0, metavar="L",
                    help="only time the backbone step at KV length L (one JSON line; for per-context profiles)")
    ap.add_argument("--no-batched", action="store_true", help="skip the batch-8 ragged-context figure")
    ap.add_argument("--no-prefill", action="store_true", help="skip the MFMA prefill figures")
    ap.add_argument("--no-contexts", action="store_true", help="skip the backbone figures at L=129 and L=2048")
    ap.add_argument("--prefill-only", action="store_true", help="only the MFMA prefill figures (one JSON line)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device-to-device copies of MIB MiB (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X "
              "(batch-1 decode of one stream runs on a single GPU; streams shard one per GPU)", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__ as ge
    pkg = ge.import_package()
    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 5}), flush=True)
        return

    sd = pkg.synthetic_state_dict(seed=1234, device="cuda")
    bbg = pkg.TTSMegakernelGenerator(model=sd, max_seq_len=4096)
    if args.backbone_context:
        print(json.dumps({"backbone": backbone_figure(bbg, args.backbone_context, steps=args.steps,
                                                      warmup=args.warmup)}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_figures(bbg)}), flush=True)
        return
    cpg = pkg.CodePredictorMegakernelGenerator(model=sd, max_seq_len=32)
    bb, cp = bbg.decoder, cpg.decoder
    g = torch.Generator(device="cuda").manual_seed(5)
    k = torch.randn(28, 8, 511, 128, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(28, 8, 511, 128, generator=g, device="cuda").to(torch.bfloat16)
    bb.set_kv_cache(k, v)
    del k, v
    i32 = dict(dtype=torch.int32, device="cuda")
    g0 = torch.tensor([17], **i32)
    done = torch.zeros(1, **i32)
    hist = torch.zeros(1, **i32)
    toks = torch.zeros(16, **i32)
    comb = torch.empty(1024, dtype=torch.bfloat16, device="cuda")
    text = torch.randn(1024, generator=g, device="cuda").to(torch.bfloat16)
    bb.set_position(511)
    bb.decode_step_select(text, g0, hist, 0, 1.0, -1, False, False, 1.0, 0, 1.0, 0, 0)
    hidden = bb.hidden_state_buffer()

    def one_frame(step):
        cp.frame(hidden, g0, text, toks, comb, -1, done, False, 1.0, 0, 1.0, 0, step)
        bb.set_position(511)
        bb.decode_step_select(comb, g0, hist, 0, 1.0, -1, False, False, 1.0, 0, 1.0, 0, step + 1)

    for i in range(args.warmup):
        one_frame(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        one_frame(args.warmup + i)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    bb.check_error()
    cp.check_error()

    # per-kernel durations with HIP events on the launch stream (torch's current stream)
    n_ev = 30
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n_ev)]
    for i in range(n_ev):
        ev[i][0].record()
        cp.frame(hidden, g0, text, toks, comb, -1, done, False, 1.0, 0, 1.0, 0, i)
        ev[i][1].record()
        bb.set_position(511)
        bb.decode_step_select(comb, g0, hist, 0, 1.0, -1, False, False, 1.0, 0, 1.0, 0, i + 1)
        ev[i][2].record()
    torch.cuda.synchronize()
    t_cp = sum(e[0].elapsed_time(e[1]) for e in ev) / n_ev * 1e-3
    t_bb = sum(e[1].elapsed_time(e[2]) for e in ev) / n_ev * 1e-3
    cp_gbs = cp_frame_bytes() / t_cp / 1e9
    bb_gbs = backbone_bytes(512) / t_bb / 1e9
    dominant = ("qtts_decode_kernel<false, false> (code-predictor frame)", cp_gbs, cp_frame_bytes(), PMC_TRAFFIC["cp_frame"]) \
        if t_cp >= t_bb else \
        ("qtts_decode_kernel<true, false> (backbone step, L=512)", bb_gbs, backbone_bytes(512), PMC_TRAFFIC["backbone_step"])

    fps = args.steps / el
    out = {
        "metric": "codec frames/s (1 backbone+15 CP steps), bs=1; % HBM roofline",
        "value": round(fps, 2),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000 * el / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 weights; f64 accumulation (backbone), f32 (code predictor)",
        "data": "synthetic (seeded random-init weights, random bf16 KV cache)",
        "config": {"workload": "codec frame at 512 context: backbone 28 layers (L=512) + code predictor "
                               "5 layers x 16 positions, 15 lm-heads; batch 1 (BASELINE configs[2] frame)",
                   "global_batch": 1, "seq_len": 512, "parallelism": "none (1 GPU)"},
        "frame_roofline_frac": round(fps * frame_bytes(512) / (HBM_PEAK_GBS * 1e9), 4),
        "kernels_us": {"cp_frame": round(t_cp * 1e6, 2), "backbone_step": round(t_bb * 1e6, 2)},
        "backbone_steps_per_s": round(1.0 / t_bb, 1),
        "backbone_roofline_frac": round(bb_gbs / HBM_PEAK_GBS, 4),
        "cp_steps_per_s": round(15.0 / t_cp, 1),
        "cp_roofline_frac": round(cp_gbs / HBM_PEAK_GBS, 4),
        "kernel_gbs": {"cp_frame": round(cp_gbs, 1), "backbone_step": round(bb_gbs, 1)},
        "roofline": {"bound": "hbm", "kernel": dominant[0], "achieved": round(dominant[1], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dominant[1] / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": dominant[2], "traffic": dominant[3]},
    }
    # backbone steps/s and roofline at config 0's context (L = 129) and config 3's (L = 2048)
    if not args.no_contexts:
        out["backbone_by_context"] = {f"L{L}": backbone_figure(bbg, L) for L in (129, 2048)}
    # the prefill is timed before the batched phase, whose 8 stream decoders stay allocated until
    # it returns (with them alive, the 229 host launches of a 128-token prefill fell behind the GPU)
    if not args.no_prefill:
        out["prefill"] = prefill_figures(bbg)
    if not args.no_batched:
        out["batched_c4"] = batched_c4(pkg, sd)
    # the decoders and their device memory are released before the CPU leg and before exit,
    # with the device idle, so nothing device-side is left to the interpreter's teardown
    del bb, cp, bbg, cpg, hidden
    torch.cuda.synchronize()
    pkg._ext.load().shutdown()
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(max(10, args.cpu_runs))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
