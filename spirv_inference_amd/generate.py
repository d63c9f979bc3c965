"""Greedy TinyLlama-shape generation from seeded prompt ids (command line).

The role of the reference's decode driver (source/xla_hlo/tools/run_llama_spirv.py:194-295:
feed the prompt, then append argmax tokens one step at a time), on the resident KV-cache
decoder: the prompt is fed one step per id, then `--tokens` greedy tokens are generated in one
decode call of the selected engine.  Weights are the seeded random-init ones (no checkpoint),
so the token ids are only meaningful for parity and timing.

    python -m spirv_inference_amd.generate --tokens 20 --repeat 3

prints the generated ids and the decode time per token of each repetition.  Real weights
supplied locally replace the seeded ones: `--reference-fixture DIR` (export_llama.py's
raw-f32 parameter files) or `--safetensors FILE` (a Hugging Face checkpoint).  With
`--profile-phases N` it also decodes N tokens in one persistent launch with the in-kernel phase
stamps on and prints, for the last of them, the time each workgroup spends in the phases of a
layer and at the grid barriers between them (means over workgroups, summed over layers).
"""
from __future__ import annotations

import argparse
import ctypes as C
import time

import numpy as np

from ._lib import check, lib
from .models import TINYLLAMA, Llama
from .runtime import Context

PHASES = ("A rmsnorm+qkv", "B1 attention", "B2 wo+residual", "C rmsnorm+gate/up", "D down+residual")


def phase_profile(lm: Llama, n: int) -> str:
    """Per-phase work and barrier time of the last of n tokens decoded in one persistent launch
    (shp_llama_profile_persistent stamps every workgroup at each grid barrier: arrival, exit)."""
    n_layers = TINYLLAMA["n_layers"]
    nb = 5 * n_layers + 1
    cap = n * nb * 16 * 512  # room for up to 512 workgroups (one per CU)
    buf = (C.c_ulonglong * cap)()
    grid = C.c_int32()
    check(lib().shp_llama_profile_persistent(C.c_void_p(lm.handle), n, buf, C.c_uint64(cap),
                                             C.byref(grid)), "shp_llama_profile_persistent")
    g = grid.value
    a = np.frombuffer(buf, dtype=np.uint64)[: n * nb * 16 * g].reshape(n, nb, 16, g)
    a = a.astype(np.int64)
    tick_us = 0.01  # wall_clock64 runs at 100 MHz
    it = n - 1
    prev = a[it - 1, nb - 1, 1] if it > 0 else a[it, 0, 0]
    start = prev.max()
    work = {k: 0.0 for k in PHASES + ("E lm_head+argmax",)}
    bar = dict.fromkeys(work, 0.0)
    for kb in range(nb):
        name = PHASES[kb % 5] if kb < 5 * n_layers else "E lm_head+argmax"
        arrive, leave = a[it, kb, 0], a[it, kb, 1]
        work[name] += float(((arrive - prev) * tick_us).mean())
        bar[name] += float(((leave - arrive) * tick_us).mean())
        prev = leave
    span = float((a[it, nb - 1, 1].max() - start) * tick_us)
    lines = [f"token {it} of {n}, {g} workgroups, span {span:.1f} us",
             "| phase | work us / token | barrier us / token |", "|---|---|---|"]
    lines += [f"| {k} | {work[k]:.1f} | {bar[k]:.1f} |" for k in work]
    lines.append(f"total work {sum(work.values()):.1f} us, barriers {sum(bar.values()):.1f} us")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--prompt-tokens", type=int, default=32)
    ap.add_argument("--tokens", type=int, default=20)
    ap.add_argument("--repeat", type=int, default=1)
    ap.add_argument("--seed", type=int, default=2, help="weight seed")
    ap.add_argument("--prompt-seed", type=int, default=3)
    ap.add_argument("--engine", choices=("default", "persistent", "graph", "kernels"),
                    default="default")
    ap.add_argument("--reference-fixture", metavar="DIR",
                    help="load export_llama.py raw-f32 parameters from DIR")
    ap.add_argument("--safetensors", metavar="FILE", nargs="+",
                    help="load a Hugging Face safetensors checkpoint (one file or shards)")
    ap.add_argument("--profile-phases", type=int, default=0, metavar="N",
                    help="after the timed runs, stamp-profile N tokens of the persistent engine")
    ap.add_argument("--copy-calibration-mb", type=int, default=0, metavar="MB",
                    help="finish with a plain device copy of MB MiB (scales rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    rng = np.random.default_rng(args.prompt_seed)
    prompt = [int(t) for t in rng.integers(0, TINYLLAMA["vocab"], args.prompt_tokens)]
    with Context("any") as ctx:
        lm = Llama(ctx, seed=args.seed)
        if args.reference_fixture:
            from .weights import load_llama_reference_fixture
            load_llama_reference_fixture(lm, args.reference_fixture)
        elif args.safetensors:
            from .weights import load_llama_safetensors
            load_llama_safetensors(lm, args.safetensors)
        if args.engine != "default":
            lm.set_engine(args.engine)
        print(f"engine {lm.engine}", flush=True)
        for _ in range(args.repeat):
            lm.reset()
            for t in prompt:
                lm.step(t)
            ctx.sync()
            t0 = time.perf_counter()
            lm.decode(args.tokens)
            ctx.sync()
            dt = time.perf_counter() - t0
            toks = lm.tokens()[len(prompt) - 1:len(prompt) - 1 + args.tokens]
            print(f"{dt / args.tokens * 1e3:.3f} ms/token  tokens {toks}", flush=True)
        if args.profile_phases > 0:
            lm.reset()
            for t in prompt:
                lm.step(t)
            print(phase_profile(lm, args.profile_phases), flush=True)
        lm.close()
        if args.copy_calibration_mb > 0:
            n = args.copy_calibration_mb * (1 << 20) // 4
            src, dst = ctx.empty(n), ctx.empty(n)
            ctx.fill_random(src, 9, 0, "uniform", 0.0, 1.0)
            ctx.launch("reshape", src, None, dst, [n])
            ctx.sync()
            src.free()
            dst.free()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
