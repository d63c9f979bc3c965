#!/usr/bin/env python3
"""Benchmark of the operator-kernel hot path on one MI355X.

Headline (BASELINE.json metric): ResNet-50 v1.5 fp32 img/s at batch 32 through the HLO-path
graph, with TinyLlama-1.1B fp32 greedy decode tok/s and the
roofline fractions reported beside it.  Synthetic seeded inputs and random-init weights,
generated on the device; inputs are resident in HBM before the timed region starts.

Timed region (`value`): K b32 steps, each one replay of a hipGraph capture of the whole
forward on one HIP stream (one b32 chain), bracketed by stream synchronisation, host clock.
Profiled region: K b32 passes launched eagerly on the same stream with a hipEvent pair around
every kernel; those per-kernel durations give the roofline of the dominant kernel (the MFMA
implicit-GEMM convolution).  Reported beside the headline, not as it: throughput with
`--concurrency` independent b32 steps in flight on as many streams (extra.concurrent).
The CPU baseline is the C oracle (restated reference loops, OpenMP) timed on bounded samples
of the same workloads on this box's host cores, all cores and one thread.

Prints ONE JSON line.  --gpus N > 1 exits with an explanation (single-GPU build).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ResNet-50 fp32 img/s @b32; TinyLlama fp32 decode tok/s; % fp32-MFMA/HBM roofline"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def conv_flops(op) -> float:
    q = op.push
    if op.kernel == "hlo_conv_nhwc_hwio":
        return 2.0 * q[0] * q[7] * q[8] * q[6] * q[4] * q[5] * q[3]
    return 0.0


def conv_bytes(op) -> float:
    """Algorithmic HBM bytes of one hlo_conv_nhwc_hwio launch: input (only the sampled pixels
    for a strided 1x1), HWIO weights, output, and the residual read when the epilogue adds one."""
    q = op.push
    if op.kernel != "hlo_conv_nhwc_hwio":
        return 0.0
    n, ih, iw, ic, kh, kw, oc, oh, ow, sh, sw = q[:11]
    inp = n * oh * ow * ic if (kh == 1 and kw == 1 and (sh > 1 or sw > 1)) else n * ih * iw * ic
    out = n * oh * ow * oc
    return 4.0 * (inp + kh * kw * ic * oc + out * (2 if op.residual >= 0 else 1))


def measured_conv_traffic(batch: int):
    """HBM bytes per conv launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary of
    this workload (profiles/resnet50_b32_conv_layers.md), or None for other batch sizes."""
    path = os.path.join(ROOT, "profiles", "resnet50_b32_conv_layers.md")
    if batch != 32 or not os.path.exists(path):
        return None
    for ln in open(path):
        if ln.startswith("hbm_bytes_per_conv_launch"):
            return float(ln.split("=")[1])
    return None


def measured_config_hbm(name: str):
    """Per-family kernel time and HBM bytes of one latency config, from the committed
    rocprofv3 summary profiles/<name>.md (kernel trace + FETCH_SIZE / WRITE_SIZE passes of
    an eager forward): {registry kernel: {us, hbm_gbs, frac_hbm, hbm_over_alg}}."""
    path = os.path.join(ROOT, "profiles", name + ".md")
    if not os.path.exists(path):
        return None
    out, in_hbm = {}, False
    for ln in open(path):
        if ln.startswith("## HBM traffic"):
            in_hbm = True
            continue
        if ln.startswith("## ") and in_hbm:
            break
        if in_hbm and ln.startswith("| `"):
            c = [x.strip() for x in ln.strip().strip("|").split("|")]
            out[c[0].strip("`")] = {"us": float(c[2]), "hbm_gbs": float(c[5]),
                                    "frac_hbm": round(float(c[5]) / PEAK_HBM_GBS, 4),
                                    "hbm_over_alg": float(c[8])}
    return out or None


def measured_decode_traffic(n_prompt: int, n_new: int):
    """HBM bytes per token of the persistent decode from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/tinyllama_decode_persistent.md: 32-token prompt, 20 new
    tokens), or None for another workload."""
    path = os.path.join(ROOT, "profiles", "tinyllama_decode_persistent.md")
    if (n_prompt, n_new) != (32, 20) or not os.path.exists(path):
        return None
    for ln in open(path):
        if ln.startswith("hbm_bytes_per_token"):
            return float(ln.split("=")[1])
    return None


def time_alternating_steps(ctx, m, steps: int, warmup: int, batch: int, streams: int):
    """K b{batch} steps dealt round-robin over `streams` contexts (one HIP stream and hipGraph
    each, same weights and input), so consecutive steps overlap.  Returns (img/s, ms/step, top-1)."""
    from spirv_inference_amd import Context
    from spirv_inference_amd.models import Model
    x = m.input(0).download()
    ctxs = [ctx] + [Context("any") for _ in range(streams - 1)]
    parts = []
    try:
        for c in ctxs:
            part = Model(c, "resnet50_v1_5", batch, seed=2)
            parts.append(part)
            part.input(0).upload(x)
            part.use_graph(True)
        for _ in range(max(warmup, 1)):
            for part in parts:
                part.run()
        for c in ctxs:
            c.sync()
        t0 = time.perf_counter()
        for k in range(steps):
            parts[k % streams].run()
        for c in ctxs:
            c.sync()
        elapsed = time.perf_counter() - t0
        top1 = [int(i) for i in np.argmax(parts[-1].output(1).download().reshape(batch, -1), axis=1)]
        return batch * steps / elapsed, elapsed / steps * 1e3, top1
    finally:
        for part in parts:
            part.close()
        for c in ctxs[1:]:
            c.close()


def time_hlo_module(ctx, m, steps: int, warmup: int, batch: int):
    """The same step through the HLO path: the generated ResNet-50 v1.5 HLO text module,
    parsed, compiled (hlo_program) on the graph's own weights and input, replayed from a
    hipGraph K times (host clock).  Its output must equal the C++ graph's bit for bit."""
    from spirv_inference_amd import hlo_exec as X
    from spirv_inference_amd import hlo_gen as G
    from spirv_inference_amd.hlo_program import HloProgram
    text, spec = G.resnet50_v15(batch)
    ops = X.parse_hlo_text(text)
    m.use_graph(False)
    m.run()
    ctx.sync()
    want = m.output(0).download()
    prog = HloProgram(X.DeviceBackend(ctx), ops, G.model_bindings(m, spec))
    try:
        for _ in range(max(warmup, 2)):
            prog.run(graph=True)
        ctx.sync()
        identical = bool(np.array_equal(prog.read(0).reshape(-1), want))
        t0 = time.perf_counter()
        for _ in range(steps):
            prog.run(graph=True)
        ctx.sync()
        elapsed = time.perf_counter() - t0
        return dict(img_s=round(batch * steps / elapsed, 3),
                    ms_per_step=round(elapsed / steps * 1e3, 4), hlo_ops=len(ops),
                    launches=len(prog.launches), identical_to_cpp_graph=identical,
                    region="generated ResNet-50 v1.5 HLO text -> parse_hlo_text -> hlo_program "
                           "(fused epilogues / row kernels) -> one hipGraph, replayed K times")
    finally:
        prog.close()


def bench_resnet(ctx, steps: int, warmup: int, batch: int, concurrency: int = 1):
    from spirv_inference_amd.models import Model
    m = Model(ctx, "resnet50_v1_5", batch, seed=2)
    flops, wbytes = m.work()
    ops = m.ops()
    cflops = sum(conv_flops(o) for o in ops)
    cbytes = sum(conv_bytes(o) for o in ops)
    n_conv = sum(1 for o in ops if o.kernel == "hlo_conv_nhwc_hwio")
    # timed region: the step captured once into a hipGraph and replayed K times
    m.use_graph(True)
    for _ in range(warmup):
        m.run()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.run()
    ctx.sync()
    t1 = time.perf_counter()
    elapsed = t1 - t0
    # profiled region: the same K steps launched eagerly with a hipEvent pair around every
    # kernel on the context stream -> per-kernel durations for the roofline
    m.use_graph(False)
    m.run()
    ctx.sync()
    ctx.timing(True)
    ctx.timing_reset()
    e0 = time.perf_counter()
    for _ in range(steps):
        m.run()
    ctx.sync()
    e1 = time.perf_counter()
    rep = ctx.timing_report()
    ctx.timing(False)
    conv_ms, conv_n = rep.get("hlo_conv_nhwc_hwio", (0.0, 0))
    kernel_ms = sum(v[0] for v in rep.values()) / steps
    logits = m.output(1).download().reshape(batch, -1)
    top1 = [int(i) for i in np.argmax(logits, axis=1)]
    achieved = cflops * steps / (conv_ms / 1e3) / 1e12 if conv_ms > 0 else 0.0
    res = dict(
        img_s=batch * steps / elapsed, ms_per_step=elapsed / steps * 1e3,
        eager_ms_per_step=(e1 - e0) / steps * 1e3, kernel_ms_per_step=kernel_ms,
        flops_per_img=flops / batch, conv_flops_per_step=cflops, conv_bytes_per_step=cbytes, n_conv=n_conv,
        conv_ms_per_step=conv_ms / steps, conv_launches=conv_n,
        conv_avg_launch_ms=conv_ms / max(conv_n, 1), achieved_tflops=achieved,
        per_kernel_ms={k: v[0] / steps for k, v in sorted(rep.items())}, top1=top1,
        weight_bytes=wbytes, concurrent=None)
    res["hlo_path"] = time_hlo_module(ctx, m, steps, warmup, batch)
    if concurrency > 1:
        img_s, ms, top1_c = time_alternating_steps(ctx, m, steps, warmup, batch, concurrency)
        res["concurrent"] = dict(streams=concurrency, img_s=round(img_s, 3),
                                 ms_per_step=round(ms, 4), top1_identical=top1_c == top1,
                                 region=f"K b{batch} steps dealt round-robin over {concurrency} "
                                        "contexts (one HIP stream and hipGraph each), so up to "
                                        f"{concurrency} independent b{batch} steps are in "
                                        "flight; host clock")
    m.close()
    return res


def bench_config(ctx, arch: str, batch: int, seq_len: int, steps: int):
    """Latency of one graph-replayed forward of another benchmark config, with its dense
    FLOPs (2 x MAC of the convolutions and dots) against the fp32 MFMA peak."""
    from spirv_inference_amd.models import Model
    m = Model(ctx, arch, batch, seq_len, seed=2)
    flops, wbytes = m.work()
    m.use_graph(True)
    for _ in range(3):
        m.run()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.run()
    ctx.sync()
    ms = (time.perf_counter() - t0) / steps * 1e3
    cnn = arch in ("mobilenet_v2", "efficientnet_lite0")
    tfl = time_tflite_executor(ctx, m, steps) if cnn else None
    fused = sum(op.kernel == "inverted_residual_nhwc" for op in m.ops())
    m.close()
    tflops = flops / (ms / 1e3) / 1e12
    out = {"batch": batch, "seq_len": seq_len or None, "ms_per_forward": round(ms, 4),
           "gflop_per_forward": round(flops / 1e9, 3), "weight_mb": round(wbytes / 1e6, 2),
           "achieved_tflops": round(tflops, 3),
           "frac_fp32_mfma": round(tflops / PEAK_FP32_MFMA_TFLOPS, 4),
           "tflite_executor": tfl}
    if cnn:  # the same graph with every MBConv block as the TFLite scheduler's three operators
        from spirv_inference_amd import Context
        with Context("any") as c3:
            c3.tune("ir_fuse", -1)
            m3 = Model(c3, arch, batch, seq_len, seed=2)
            m3.use_graph(True)
            for _ in range(3):
                m3.run()
            c3.sync()
            t0 = time.perf_counter()
            for _ in range(steps):
                m3.run()
            c3.sync()
            out["mbconv_blocks_fused"] = fused
            out["three_operator_ms_per_forward"] = round((time.perf_counter() - t0) / steps * 1e3, 4)
            m3.close()
    return out


def time_tflite_executor(ctx, m, steps: int):
    """The same forward through the TFLite front end: the resident graph exported to a TFL3
    file, parsed, and run by TfliteExecutor on the graph's input, eagerly (one ctypes launch
    per op from Python) and replayed from the executor's hipGraph (host clock, K
    forwards each).  Its output must equal the graph's bit for bit."""
    from spirv_inference_amd import tflite as T
    m.run()
    ctx.sync()
    want = m.output(0).download()
    model = T.parse_model(T.model_to_tflite(m))
    ex = T.TfliteExecutor(ctx, model)
    try:
        ex.set_input(m.input(0).download())
        out = {}
        for mode in ("eager", "graph"):
            for _ in range(3):
                ex.run(graph=mode == "graph")
            ctx.sync()
            t0 = time.perf_counter()
            for _ in range(steps):
                ex.run(graph=mode == "graph")
            ctx.sync()
            out[f"{mode}_ms_per_forward"] = round((time.perf_counter() - t0) / steps * 1e3, 4)
        out["identical_to_graph"] = bool(ex.output().tobytes() == want.tobytes())
        out["operators"] = len(model.operators)
        out["launches"] = sum(len(o["dispatches"]) for o in ex.op_log)
        out["region"] = ("the graph exported to TFL3 -> parse_model -> TfliteExecutor; eager: "
                         "one launch per op from Python; graph: one hipGraph replay per forward")
        return out
    finally:
        ex.close()


def bench_elementwise(ctx, elems: int = 64 << 20, reps: int = 20):
    """HBM rate of the elementwise stream kernels (north star: >= 70 % of HBM for elementwise):
    a copy (the `reshape` kernel) and an `add` over 256 MiB float tensors, timed with a hipEvent
    pair per launch.  Bytes = every operand read once + the output written once."""
    a, b, c = ctx.empty(elems), ctx.empty(elems), ctx.empty(elems)
    out = {}
    for name, nin in (("reshape", 1), ("add", 2)):
        for _ in range(3):
            ctx.launch(name, a, b if nin == 2 else None, c, [elems])
        ctx.sync()
        ctx.timing(True)
        ctx.timing_reset()
        for _ in range(reps):
            ctx.launch(name, a, b if nin == 2 else None, c, [elems])
        ctx.sync()
        rep = ctx.timing_report()
        ctx.timing(False)
        sec = sum(v[0] for v in rep.values()) / reps / 1e3
        gbs = 4.0 * elems * (nin + 1) / sec / 1e9
        out["copy" if name == "reshape" else name] = {
            "kernel": name, "bytes_per_launch": 4 * elems * (nin + 1), "us": round(sec * 1e6, 2),
            "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4)}
    for t in (a, b, c):
        t.free()
    return out


def time_decode(ctx, lm, prompt, n_new: int):
    lm.reset()
    for t in prompt:
        lm.step(t)
    ctx.sync()
    t0 = time.perf_counter()
    lm.decode(n_new)
    ctx.sync()
    t1 = time.perf_counter()
    toks = lm.tokens()
    return (t1 - t0) / n_new, toks[len(prompt) - 1:len(prompt) - 1 + n_new]


def bench_decode(ctx, n_new: int, n_prompt: int):
    from spirv_inference_amd.models import TINYLLAMA, Llama
    rng = np.random.default_rng(3)
    prompt = [int(t) for t in rng.integers(0, TINYLLAMA["vocab"], n_prompt)]
    lm = Llama(ctx, seed=2)
    engine = lm.engine  # the default: persistent where the device allows it
    wbytes = lm.weight_bytes()
    # the per-op engine (one hipGraph per token) for comparison, then the default engine
    lm.set_engine("graph")
    time_decode(ctx, lm, prompt, 2)
    graph_s, graph_gen = time_decode(ctx, lm, prompt, n_new)
    lm.set_engine(engine)
    time_decode(ctx, lm, prompt, 2)
    s_per_tok, gen = time_decode(ctx, lm, prompt, n_new)
    cfg = TINYLLAMA
    # KV bytes read per token: K and V of every layer for positions 0..pos
    kv_tok = [2 * cfg["n_layers"] * cfg["n_kv_heads"] * 64 * 4 * (p + 1)
              for p in range(n_prompt, n_prompt + n_new)]
    # every weight is streamed once per token except the embedding table, of which one row
    # is read
    embed_bytes = cfg["vocab"] * cfg["hidden"] * 4.0
    bytes_tok = wbytes - embed_bytes + cfg["hidden"] * 4.0 + float(np.mean(kv_tok))
    return dict(tok_s=1.0 / s_per_tok, ms_per_token=s_per_tok * 1e3, bytes_per_token=bytes_tok,
                achieved_gbs=bytes_tok / s_per_tok / 1e9, prompt=prompt, tokens=gen, lm=lm,
                engine=engine, graph_tok_s=1.0 / graph_s, graph_tokens_match=graph_gen == gen)


def cpu_model() -> str:
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_model(ctx, arch: str, sample: int, seq_len: int = 0, gpu_top1=None):
    """Oracle forward of the first `sample` inputs of a config's batch: inputs and weights
    depend only on (seed, tensor id, element index), so a batch-`sample` graph holds exactly
    those inputs of the full batch."""
    from oracle import walk
    from spirv_inference_amd.models import Model
    m = Model(ctx, arch, sample, seq_len, seed=2)
    host = walk.load_constants(m)
    t0 = time.perf_counter()
    out = walk.chained(m, host)
    t1 = time.perf_counter()
    res = dict(value=sample / (t1 - t0), seconds=t1 - t0, sample=sample)
    if gpu_top1 is not None:
        logits = out[m.ops()[-2].out].reshape(sample, -1)
        top1 = [int(i) for i in np.argmax(logits, axis=1)]
        res.update(top1=top1, top1_match=top1 == list(gpu_top1[:sample]))
    m.close()
    return res


def cpu_baseline_decode(dec, n_steps: int):
    """The oracle's KV-cache decode of n_steps tokens after the same prompt (the cache is
    built untimed), on the decoder's own weights."""
    import oracle
    from spirv_inference_amd.models import TINYLLAMA
    lm = dec["lm"]
    cfg = TINYLLAMA
    c = oracle.LlamaCfg(**cfg)
    names = ("attn_norm", "wqkv", "wo", "ffn_norm", "w_gate_up", "w_down")
    layers = [[lm.weight(l, n) for n in names] for l in range(cfg["n_layers"])]
    emb, fn, head = lm.weight(0, "embed"), lm.weight(0, "final_norm"), lm.weight(0, "lm_head")
    cache = cfg["n_layers"] * cfg["n_kv_heads"] * cfg["max_seq"] * 64
    kc, vc = np.zeros(cache, np.float32), np.zeros(cache, np.float32)
    prompt = dec["prompt"]
    toks, nxt = [], None
    for pos, t in enumerate(prompt):  # build the cache (not timed)
        nxt = oracle.argmax_first(oracle.llama_step(c, layers, emb, fn, head, kc, vc, pos, t))
    toks.append(nxt)
    t0 = time.perf_counter()
    for i in range(n_steps):
        pos = len(prompt) + i
        nxt = oracle.argmax_first(oracle.llama_step(c, layers, emb, fn, head, kc, vc, pos, nxt))
        toks.append(nxt)
    t1 = time.perf_counter()
    return dict(value=n_steps / (t1 - t0), seconds=t1 - t0, tokens=toks,
                tokens_match=toks == dec["tokens"][:len(toks)])


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--concurrency", type=int, default=3,
                    help="also time this many independent b32 steps in flight on as many "
                         "streams (reported in extra.concurrent, not as the headline); 1 = skip")
    ap.add_argument("--decode-tokens", type=int, default=20)
    ap.add_argument("--prompt-tokens", type=int, default=32)
    ap.add_argument("--cpu-sample", type=int, default=32, help="images for the CPU baseline")
    ap.add_argument("--cpu-decode-steps", type=int, default=19,
                    help="decode steps for the CPU baseline (after the prompt)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the MobileNetV2 / EfficientNet-Lite0 / BERT latency lines")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="also run one `reshape` copy of this many MiB (counter calibration)")
    ap.add_argument("--elementwise-only", action="store_true",
                    help="only the elementwise HBM measurement (the profiling entry of "
                         "profiles/elementwise_256mib.md); prints its JSON")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (no collectives or sharding); "
              "run it with --gpus 1", file=sys.stderr)
        return 2

    from spirv_inference_amd import Context
    ctx = Context("any")
    log(f"device {ctx.device_name}")
    if args.elementwise_only:
        print(json.dumps({"elementwise": bench_elementwise(ctx)}), flush=True)
        return 0
    rn = bench_resnet(ctx, args.steps, args.warmup, args.batch, args.concurrency)
    log(f"resnet50 b{args.batch} (one chain): {rn['img_s']:.1f} img/s, "
        f"{rn['ms_per_step']:.3f} ms/step (eager+events {rn['eager_ms_per_step']:.3f} ms), "
        f"conv {rn['achieved_tflops']:.1f} TFLOP/s")
    hp = rn["hlo_path"]
    log(f"resnet50 b{args.batch} via the HLO text module: {hp['img_s']:.1f} img/s "
        f"({hp['launches']} launches for {hp['hlo_ops']} HLO ops; output identical to the "
        f"C++ graph: {hp['identical_to_cpp_graph']})")
    if rn["concurrent"]:
        cc = rn["concurrent"]
        log(f"resnet50 b{args.batch}, {cc['streams']} steps in flight on {cc['streams']} "
            f"streams: {cc['img_s']:.1f} img/s (top-1 identical {cc['top1_identical']})")
    configs = {}
    if not args.no_configs:
        for arch, b, sl in (("mobilenet_v2", 1, 0), ("efficientnet_lite0", 8, 0),
                            ("bert_base", 8, 128)):
            configs[arch] = bench_config(ctx, arch, b, sl, max(args.steps, 10))
            c = configs[arch]
            log(f"{arch} b{b}: {c['ms_per_forward']:.3f} ms/forward, "
                f"{c['achieved_tflops']:.1f} TFLOP/s ({100 * c['frac_fp32_mfma']:.1f}% of fp32 MFMA)")
            if "three_operator_ms_per_forward" in c:
                log(f"{arch} b{b}: {c['mbconv_blocks_fused']} MBConv blocks fused; with every "
                    f"block as three launches {c['three_operator_ms_per_forward']:.3f} ms/forward")
            if c["tflite_executor"]:
                t = c["tflite_executor"]
                log(f"{arch} b{b} via the TFLite executor: {t['graph_ms_per_forward']:.3f} ms "
                    f"(hipGraph), {t['eager_ms_per_forward']:.3f} ms (eager); output identical "
                    f"to the graph: {t['identical_to_graph']}")
    dec = None
    if not args.no_decode:
        dec = bench_decode(ctx, args.decode_tokens, args.prompt_tokens)
        log(f"tinyllama decode ({dec['engine']}): {dec['tok_s']:.1f} tok/s, "
            f"{dec['achieved_gbs']:.0f} GB/s; graph engine {dec['graph_tok_s']:.1f} tok/s "
            f"(tokens identical {dec['graph_tokens_match']})")
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    cpu = cpu1 = cpu_dec = cpu_dec1 = None
    cpu_cfg = {}
    if not args.no_cpu_baseline:
        import oracle
        oracle.set_threads(cores)
        cpu = cpu_baseline_model(ctx, "resnet50_v1_5", args.cpu_sample, gpu_top1=rn["top1"])
        log(f"cpu oracle resnet: {cpu['value']:.3f} img/s on {cores} threads "
            f"(top1 match {cpu['top1_match']})")
        for arch, sample, sl in (("mobilenet_v2", 1, 0), ("efficientnet_lite0", 8, 0),
                                 ("bert_base", 1, 128)):
            r = cpu_baseline_model(ctx, arch, sample, sl)
            cpu_cfg[arch] = {"ms_per_input": round(r["seconds"] / sample * 1e3, 2),
                             "sample": f"{sample} of the config's inputs, {cores} threads"}
            log(f"cpu oracle {arch}: {r['seconds'] / sample * 1e3:.1f} ms per input")
        if dec is not None:
            cpu_dec = cpu_baseline_decode(dec, args.cpu_decode_steps)
            log(f"cpu oracle decode: {cpu_dec['value']:.3f} tok/s "
                f"(tokens match {cpu_dec['tokens_match']})")
        oracle.set_threads(1)
        cpu1 = cpu_baseline_model(ctx, "resnet50_v1_5", 1, gpu_top1=rn["top1"])
        log(f"cpu oracle resnet, 1 thread: {cpu1['value']:.3f} img/s")
        if dec is not None:
            cpu_dec1 = cpu_baseline_decode(dec, 3)
            log(f"cpu oracle decode, 1 thread: {cpu_dec1['value']:.3f} tok/s")
        oracle.set_threads(cores)

    elementwise = bench_elementwise(ctx)
    log("elementwise: " + ", ".join(f"{k} {v['achieved']:.0f} GB/s ({100 * v['frac']:.1f} %)"
                                   for k, v in elementwise.items()))
    traffic = measured_conv_traffic(args.batch)
    host_cpu = cpu_model()
    line = {
        "metric": METRIC,
        "value": round(rn["img_s"], 3),
        "unit": "img/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(rn["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"ResNet-50 v1.5 fp32 inference, batch {args.batch}, NHWC "
                        f"{args.batch}x224x224x3 N(0,1), HLO path (hlo_conv_nhwc_hwio, "
                        "reduce_window max-pool, mean pool, dot 2048->1000, softmax), "
                        "He-normal weights (the last 1x1 conv of each bottleneck at 0.2x He, "
                        "its folded-BN gamma), folded BN as a bias N(0,0.01); one b32 chain",
            "global_batch": args.batch,
            "streams": 1,
            "flops_per_img": rn["flops_per_img"],
            "seed": 2,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "hlo_conv_nhwc_hwio (fp32 MFMA implicit GEMM)",
            "achieved": round(rn["achieved_tflops"], 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(rn["achieved_tflops"] / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": traffic,
            "traffic_unit": "HBM bytes per conv launch (rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0, "
                            "scaled by a 256 MiB copy; profiles/resnet50_b32_conv_layers.md)",
            "algorithmic_bytes_per_launch": round(rn["conv_bytes_per_step"] / rn["n_conv"]),
            "algorithmic_flops_per_step": rn["conv_flops_per_step"],
            "launches_per_step": rn["n_conv"],
            "avg_launch_ms": round(rn["conv_avg_launch_ms"], 5),
        },
        "cpu_baseline": None if cpu is None else {
            "value": round(cpu["value"], 4), "unit": "img/s", "cores": cores, "kind": "port",
            "cpu": host_cpu,
            "sample": f"C oracle (reference kernel loops, OpenMP) forward of images 0..{args.cpu_sample - 1} "
                      f"of the same b{args.batch} workload, {cpu['seconds']:.2f} s; "
                      f"top-1 identical to the GPU's: {cpu['top1_match']}",
            "one_thread": None if cpu1 is None else {
                "value": round(cpu1["value"], 4), "unit": "img/s", "cores": 1,
                "sample": f"image 0, {cpu1['seconds']:.2f} s; top-1 identical: "
                          f"{cpu1['top1_match']}"},
            "configs": cpu_cfg,
        },
        "extra": {
            "timed_region": "hipGraph replay of the whole b32 step on one HIP stream, K times, "
                            "host clock",
            "profiled_region": f"K b{args.batch} steps launched eagerly on one stream with a "
                               "hipEvent pair per kernel (roofline source)",
            "concurrent": rn["concurrent"],
            "hlo_path": rn["hlo_path"],
            "eager_ms_per_step": round(rn["eager_ms_per_step"], 4),
            "kernel_ms_per_step": round(rn["kernel_ms_per_step"], 4),
            "per_kernel_ms_per_step": {k: round(v, 4) for k, v in rn["per_kernel_ms"].items()},
            "top1": rn["top1"],
            "configs": configs,
            "configs_hbm_by_kernel": {k: measured_config_hbm(f) for k, f in (
                ("mobilenet_v2", "mobilenet_v2_b1"), ("efficientnet_lite0", "efficientnet_lite0_b8"),
                ("bert_base", "bert_base_b8_s128"))},
            "configs_hbm_source": "rocprofv3 FETCH_SIZE/WRITE_SIZE of an eager forward per config, "
                                  "profiles/<config>.md",
            "elementwise": elementwise,
        },
    }
    if dec is not None:
        line["decode"] = {
            "workload": "TinyLlama-1.1B-shape fp32 greedy decode, batch 1, 22 layers, hidden 2048, "
                        "32q/4kv heads, SwiGLU 5632, vocab 32000, N(0,0.02) weights, RMSNorm "
                        f"weights 1, {args.prompt_tokens} seeded prompt ids, {args.decode_tokens} "
                        "new tokens (KV cache; timed: one decode call of the default engine)",
            "value": round(dec["tok_s"], 3), "unit": "tok/s",
            "ms_per_token": round(dec["ms_per_token"], 4),
            "roofline": {"bound": "hbm", "achieved": round(dec["achieved_gbs"], 1),
                         "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(dec["achieved_gbs"] / PEAK_HBM_GBS, 4),
                         "traffic": (measured_decode_traffic(args.prompt_tokens, args.decode_tokens)
                                     if dec["engine"] == "persistent" else None),
                         "traffic_unit": "HBM bytes per token (rocprofv3 FETCH_SIZE x2.0 + "
                                         "WRITE_SIZE x1.0, scaled by a 256 MiB copy; "
                                         "profiles/tinyllama_decode_persistent.md)",
                         "bytes_per_token": dec["bytes_per_token"]},
            "tokens": dec["tokens"],
            "engine": dec["engine"],
            "graph_engine_tok_s": round(dec["graph_tok_s"], 3),
            "graph_engine_tokens_identical": dec["graph_tokens_match"],
            "cpu_baseline": None if cpu_dec is None else {
                "value": round(cpu_dec["value"], 4), "unit": "tok/s", "cores": cores,
                "kind": "port", "cpu": host_cpu,
                "sample": f"C oracle KV-cache decode of {args.cpu_decode_steps} tokens after the "
                          f"same prompt, {cpu_dec['seconds']:.2f} s; tokens identical to the "
                          f"GPU's: {cpu_dec['tokens_match']}",
                "one_thread": None if cpu_dec1 is None else {
                    "value": round(cpu_dec1["value"], 4), "unit": "tok/s", "cores": 1,
                    "sample": f"3 tokens, {cpu_dec1['seconds']:.2f} s"}},
        }
        dec["lm"].close()
    if args.copy_calibration_mb > 0:
        # a plain copy of known size, so FETCH_SIZE / WRITE_SIZE counters can be scaled
        n = args.copy_calibration_mb * (1 << 20) // 4
        src, dst = ctx.empty(n), ctx.empty(n)
        ctx.fill_random(src, 9, 0, "uniform", 0.0, 1.0)
        ctx.launch("reshape", src, None, dst, [n])
        ctx.sync()
        src.free()
        dst.free()
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
