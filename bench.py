"""Decode-step benchmark: device us/step and tok/s of the MI355X task-graph
decoder vs the 1.19 GB HBM weight floor.

Workload (config C3, the headline case of the metric): Qwen3-0.6B
geometry, random-init bf16 weights (seed 0), batch 1, one random start token,
greedy decode with the token fed back on the device (no host round trip), so
the context grows 1 -> K. A "step" is one decode step of the batch. Timed: K
back-to-back steps on one stream between a synchronize on each side, after W
warmup steps (the state is reset to the start token before the timed run).

Printed JSON line (one): value = tok/s (= batch * K / time); roofline = the
persistent decode kernel's algorithmic bytes per launch over its average
launch duration from HIP events recorded around every launch of the timed
region (same stream); cpu_baseline = the CPU oracle timed on a bounded sample
on this host. Extra keys: per-mode and per-batch ("sweep") device us/step of
the persistent kernel vs the captured per-op hipGraph, same kernels, at short
context and ("sweep_long_c5") at the C5 long contexts.

One GPU only: --gpus N > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "decode-fusion-boundary_amd"))
sys.path.insert(0, ROOT)

WEIGHT_BYTES = 1_192_099_840           # model_spec.QWEN3_06B.weight_bytes()
KV_BYTES_PER_POS = 114_688             # 28 layers * (K+V) * 1024 * 2 B
EMBED_ROW_BYTES = 2048
HBM_PEAK_GBPS = 8000.0
VOCAB = 151936


def step_bytes(contexts: list[int]) -> int:
    """Algorithmic HBM bytes of one decode step: all weights once, each row's KV
    (ctx positions incl. the new one) read, its new K/V written, its embedding row."""

    return WEIGHT_BYTES + sum(KV_BYTES_PER_POS * c + KV_BYTES_PER_POS + EMBED_ROW_BYTES for c in contexts)


def progress(what: str) -> None:
    """One line on stderr per phase (a long default run shows it is alive)."""
    print(f"bench: {what}", file=sys.stderr, flush=True)


def build_decoder(num_layers=28, num_blocks=64, launch="persistent", variant="tagged", fusion_groups=1,
                  attn_splits=1, **options):
    import torch
    from nanovllm.backends.megakernel.taskgraph import TaskGraphDecoder
    from nanovllm.backends.megakernel.weights import weights_from_synthetic
    from nanovllm.synthetic import make_weights

    synth = make_weights(seed=0, num_layers=num_layers)
    w = weights_from_synthetic(synth, device="cuda")
    kv = torch.zeros(2, num_layers, num_blocks, 256, 8, 128, dtype=torch.bfloat16, device="cuda")
    dec = TaskGraphDecoder(w, k_cache=kv[0], v_cache=kv[1], block_size=256, num_cache_blocks=num_blocks,
                           max_model_len=2048, launch=launch, persistent_variant=variant,
                           fusion_groups=fusion_groups, attn_splits=attn_splits, **options)
    return synth, w, kv, dec


def ragged_tables(start_ctx: list[int], steps: int, num_blocks: int, block_size: int = 256, cols: int = 8,
                  seed: int = 0) -> list[list[int]]:
    """Block tables drawn from a shuffled page pool (rows own scattered, non-contiguous
    pages); each row gets the pages its context reaches, the rest of its row is 0."""

    import random

    rng = random.Random(seed)
    pool = list(range(num_blocks))
    rng.shuffle(pool)
    tables = []
    for c in start_ctx:
        need = (c + steps + block_size - 1) // block_size  # positions c .. c+steps-1
        assert need <= cols and len(pool) >= need, "page pool too small for the workload"
        tables.append([pool.pop() for _ in range(need)] + [0] * (cols - need))
    return tables


def time_decode(dec, batch: int, start_ctx: list[int], steps: int, warmup: int, mode: str, seed: int = 0,
                per_launch_events: bool = False, tables=None):
    """Returns (seconds for `steps` steps, per-launch durations in ms or None, contexts per step).
    `tables` (list of rows) overrides the default contiguous block tables."""

    import torch

    gen = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, VOCAB, (batch,), generator=gen, dtype=torch.int64).cuda()
    pos = torch.tensor(start_ctx, dtype=torch.int64).cuda()
    pages = 8
    if tables is None:
        tables = [[b * pages + j for j in range(pages)] for b in range(batch)]
    tables = torch.tensor(tables, dtype=torch.int32).cuda()
    max_ctx = max(start_ctx) + max(steps, warmup) + 1
    run = dec.prepare_steps(batch, max_ctx, mode=mode)
    dec.stage_rows(ids, pos, tables)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    dec.check_device_error()
    dec.stage_rows(ids, pos, tables)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    events = []
    if per_launch_events:
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        if per_launch_events:
            events[i][0].record(stream)
        run()
        if per_launch_events:
            events[i][1].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    dec.check_device_error()
    durs = [a.elapsed_time(b) for a, b in events] if per_launch_events else None
    contexts = [[c + 1 + i for c in start_ctx] for i in range(steps)]
    return elapsed, durs, contexts


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(sample_steps: int = 10):
    """The CPU oracle (a restatement of the reference torch decode) on this host:
    `sample_steps` greedy batch-1 steps of the full model, each timed on its own;
    value = 1 / median step time."""

    import statistics

    import torch
    from nanovllm.synthetic import make_weights
    from oracle.qwen3_oracle import Oracle

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    synth = make_weights(seed=0, num_layers=28)
    oracle = Oracle(synth)
    kc = torch.zeros(28, 2, 256, 8, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    tok = 42
    oracle.decode_step([tok], [0], [[0]], kc, vc)  # warm
    times = []
    for i in range(sample_steps):
        t0 = time.perf_counter()
        _, toks = oracle.decode_step([tok], [i + 1], [[0]], kc, vc)
        times.append(time.perf_counter() - t0)
        tok = toks[0]
    med = statistics.median(times)
    return {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "cpu_model": cpu_model(),
            "step_s": {"median": round(med, 4), "min": round(min(times), 4), "max": round(max(times), 4),
                       "stdev": round(statistics.stdev(times), 4), "n": sample_steps},
            "sample": f"{sample_steps} greedy decode steps (each timed), batch 1, ctx 2..{sample_steps + 1}, full "
                      f"28-layer model, torch CPU fp32-accumulate restatement (oracle/qwen3_oracle.py); "
                      f"value = 1 / median step time"}


PERSISTENT_KERNELS = {"lds_dma": "k_persistent2", "v1": "k_persistent",
                      "tagged": "k_persistent4"}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "pmc_traffic.json")
CSRC = os.path.join(ROOT, "decode-fusion-boundary_amd", "csrc")


def kernel_source_hash() -> str:
    """sha256 over the HIP sources of the decode library: a PMC summary is only
    used for the kernels it was measured on."""

    import hashlib

    h = hashlib.sha256()
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".h", ".hip")):
            with open(os.path.join(CSRC, name), "rb") as f:
                h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` (e.g. ``k_persistent4<1>``) from the
    committed rocprofv3 PMC summary (``bench.py --pmc-collect``: FETCH_SIZE and
    WRITE_SIZE per dispatch, scaled by a copy kernel's readings). Returns
    (bytes or None, note)."""

    try:
        with open(TRAFFIC_FILE) as f:
            pmc = json.load(f)
    except (OSError, ValueError):
        return None, "no PMC summary"
    if pmc.get("source_hash") != kernel_source_hash():
        return None, "PMC summary measured on other kernel sources (stale); rerun bench.py --pmc-collect"
    entry = pmc.get("kernels", {}).get(kernel)
    if entry is None:
        return None, f"no PMC entry for {kernel}"
    return int(entry["traffic_bytes"]), f"{TRAFFIC_FILE.split(ROOT + os.sep)[-1]} (source {pmc['source_hash']})"


def _pmc_run(counter: str, args: list[str], out_dir: str) -> dict:
    """One rocprofv3 counter pass over a child bench process; returns
    {kernel name: mean counter value per dispatch}."""

    import csv
    import glob
    import shutil
    import subprocess

    shutil.rmtree(out_dir, ignore_errors=True)
    cmd = ["timeout", "-s", "KILL", "240", "rocprofv3", "--pmc", counter, "-d", out_dir, "-o", "pmc",
           "--output-format", "csv", "--", sys.executable, os.path.abspath(__file__), *args]
    print("pmc:", " ".join(cmd), file=sys.stderr, flush=True)
    subprocess.run(cmd, check=True, cwd=ROOT, stdout=subprocess.DEVNULL)
    per_dispatch: dict[tuple[str, str], float] = {}
    for path in glob.glob(os.path.join(out_dir, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                key = (row["Kernel_Name"], row.get("Dispatch_Id", ""))
                per_dispatch[key] = per_dispatch.get(key, 0.0) + float(row["Counter_Value"])
    out: dict[str, list[float]] = {}
    for (kernel, _), v in per_dispatch.items():
        out.setdefault(kernel, []).append(v)
    return {k: sum(v) / len(v) for k, v in out.items()}


def pmc_collect(out_path: str) -> dict:
    """Measure HBM traffic per launch of the persistent kernel at batch 1, 2, 4, 8
    (C3 shape, context 1..9) with rocprofv3 FETCH_SIZE and WRITE_SIZE, each in a
    pass of its own, calibrated by a 1 GiB device copy; writes the summary JSON."""

    import re

    kargs = ["--only-kernel", "--no-sweep", "--no-cpu-baseline", "--steps", "8", "--warmup", "2",
             "--pmc-batches", "1,2,4,8"]
    base = os.path.join(ROOT, "gpurun_out", "pmc")
    fetch = _pmc_run("FETCH_SIZE", kargs, os.path.join(base, "fetch"))
    write = _pmc_run("WRITE_SIZE", kargs, os.path.join(base, "write"))
    cfetch = _pmc_run("FETCH_SIZE", ["--copy-calibration"], os.path.join(base, "fetch_copy"))
    cwrite = _pmc_run("WRITE_SIZE", ["--copy-calibration"], os.path.join(base, "write_copy"))
    copy_kib = (1 << 30) / 1024
    f_copy = max(v for k, v in cfetch.items() if "copy" in k.lower())
    w_copy = max(v for k, v in cwrite.items() if "copy" in k.lower())
    fetch_factor, write_factor = copy_kib / f_copy, copy_kib / w_copy
    kernels = {}
    for name, fk in fetch.items():
        m = re.search(r"(k_persistent\d?)<(\d)>", name)
        if not m:
            continue
        key = f"{m.group(1)}<{m.group(2)}>"
        wk = next((v for n, v in write.items() if key in n.replace(" ", "")), None)
        if wk is None:
            continue
        b = int(m.group(2))
        algorithmic = sum(step_bytes([c] * b) for c in range(1, 9)) / 8
        traffic = fk * 1024 * fetch_factor + wk * 1024 * write_factor
        kernels[key] = {"fetch_kib": round(fk, 2), "write_kib": round(wk, 2),
                        "read_bytes": int(fk * 1024 * fetch_factor), "written_bytes": int(wk * 1024 * write_factor),
                        "traffic_bytes": int(traffic), "algorithmic_bytes": int(algorithmic),
                        "traffic_over_algorithmic": round(traffic / algorithmic, 4)}
    summary = {"source_hash": kernel_source_hash(),
               "workload": "C3 shape: batch B, contexts 1..9 (8 timed steps after 2 warmup), tagged persistent kernel",
               "calibration": {"copy_bytes_each_way": 1 << 30, "fetch_kib_per_copy": round(f_copy, 2),
                               "write_kib_per_copy": round(w_copy, 2), "fetch_factor": round(fetch_factor, 4),
                               "write_factor": round(write_factor, 4)},
               "commands": [f"rocprofv3 --pmc {c} -d <dir> -o pmc --output-format csv -- python3 bench.py "
                            + " ".join(a) for c in ("FETCH_SIZE", "WRITE_SIZE")
                            for a in (kargs, ["--copy-calibration"])],
               "kernels": kernels}
    with open(out_path, "w") as f:
        json.dump(summary, f, indent=1)
    return summary


def copy_calibration(nbytes: int = 1 << 30, launches: int = 4):
    """A plain device-to-device copy of known size (read nbytes + write nbytes
    per launch) whose FETCH_SIZE/WRITE_SIZE readings calibrate the counters."""

    import torch

    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda").normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(launches):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "launches": launches}))


def long_context_runs(workload: str, steps: int, warmup: int, dec=None) -> dict:
    """C4 (batch 8, 512-token prompts) or C5 (batch 1/2/4/8, prompt lengths
    U[1024,1920], ragged block tables): device us/step of the persistent kernel
    and of the captured per-op hipGraph, same kernels, same inputs. The cache holds
    the previous run's (or zero) K/V in the prompt positions: the step's work and
    bytes do not depend on their values."""

    import random

    num_blocks = 8 * 8 + 8
    own = dec is None
    if own:
        _, _, _, dec = build_decoder(num_blocks=num_blocks)
    rng = random.Random(0)
    if workload == "c4":
        cases = [(8, [512] * 8)]
    else:
        cases = [(b, [rng.randint(1024, 1920) for _ in range(b)]) for b in (1, 2, 4, 8)]
    out = {}
    for b, start in cases:
        tables = ragged_tables(start, max(steps, warmup), num_blocks, seed=b)
        for mode in ("persistent", "graph"):
            _, durs, ctxs = time_decode(dec, b, start, steps, warmup, mode, per_launch_events=True, tables=tables)
            us = sum(durs) / len(durs) * 1e3
            nbytes = sum(step_bytes(c) for c in ctxs) / len(ctxs)
            out[f"{mode}_b{b}"] = {"us_per_step": round(us, 2), "tok_per_s": round(b / us * 1e6, 1),
                                   "GBps": round(nbytes / us / 1e3, 1),
                                   "floor_us": round(nbytes / HBM_PEAK_GBPS / 1e3, 2),
                                   "splits": dec.splits_for(max(start) + steps + 1, b, mode),
                                   "pair_heads": dec.pair_heads_for(max(start) + steps + 1, b),
                                   "ctx": [min(start) + 1, max(start) + steps]}
    if own:
        dec.close()
    return out


def fusion_sweep(steps: int, warmup: int) -> dict:
    """Layer segments per step (fusion_groups g: g persistent launches of 28/g
    layers each, the LM head in the last) at batch 1 and 8, short context."""

    import torch

    out = {}
    for g in (1, 2, 4, 7, 14, 28):
        _, _, _, dec = build_decoder(num_blocks=72, fusion_groups=g)
        for b in (1, 8):
            _, durs, ctxs = time_decode(dec, b, [0] * b, steps, warmup, "persistent", per_launch_events=True)
            us = sum(durs) / len(durs) * 1e3
            out[f"g{g}_b{b}"] = {"us_per_step": round(us, 2), "launches_per_step": g,
                                 "GBps": round(sum(step_bytes(c) for c in ctxs) / len(ctxs) / us / 1e3, 1)}
        dec.close()
        del dec
        torch.cuda.empty_cache()
    return out


def engine_runs(batch: int = 8, prompt_len: int = 512, max_tokens: int = 128) -> dict:
    """The plugin end to end: ``LLM.generate`` with ``decode_backend="megakernel"``
    and with ``"torch"`` on the same GPU (``--engine``: batch 1 with a 16-token prompt,
    and the C4 shape). It includes the torch
    prefill, the scheduler, per-step host staging and the one device-to-host read
    per step. Reports the median decode-step wall time and decode tok/s."""

    import random
    import tempfile

    import torch
    from nanovllm import LLM, SamplingParams
    from nanovllm.synthetic import write_model_dir

    rng = random.Random(0)
    prompts = [[rng.randrange(VOCAB) for _ in range(prompt_len)] for _ in range(batch)]
    sp = SamplingParams(temperature=0.0, max_tokens=max_tokens, ignore_eos=True)
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        path = write_model_dir(os.path.join(tmp, "qwen3_06b_synthetic"), num_layers=28)
        for backend in ("megakernel", "torch"):
            llm = LLM(path, max_model_len=2048, num_kvcache_blocks=8 * batch, max_num_seqs=8,
                      decode_backend=backend)
            llm.generate([p[:16] for p in prompts], SamplingParams(temperature=0.0, max_tokens=4, ignore_eos=True))
            m = llm.generate_with_metrics(prompts, sp)["metrics"]
            llm.exit()
            del llm
            torch.cuda.empty_cache()
            step = m["decode_step_median_s"]
            out[backend] = {"decode_step_median_us": round(step * 1e6, 1), "decode_tok_per_s": round(batch / step, 1),
                            "decode_steps": m["decode_steps"], "decode_backends": m["decode_backends"],
                            "fallback_reasons": m["fallback_reasons"], "wall_time_s": round(m["wall_time_s"], 3)}
    return {"batch": batch, "prompt_len": prompt_len, "max_tokens": max_tokens, **out}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mode", default="persistent", choices=["persistent", "graph", "stages"])
    ap.add_argument("--variant", default="tagged", choices=sorted(PERSISTENT_KERNELS),
                    help="persistent kernel variant")
    ap.add_argument("--only-kernel", action="store_true", help="timed loop only (for profilers)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a 1 GiB device copy only (counter calibration under rocprofv3 --pmc)")
    ap.add_argument("--attn-splits", type=int, default=1, help="minimum split-KV factor (megakernel_attn_splits)")
    ap.add_argument("--start-ctx", type=int, default=0,
                    help="cached positions per row before the first timed step (c3 path; the KV holds zeros)")
    ap.add_argument("--workload", default="c3", choices=["c3", "c4", "c5"],
                    help="c3: the headline line (default); c4/c5: long-context persistent vs hipGraph table")
    ap.add_argument("--engine", action="store_true",
                    help="LLM.generate end to end, megakernel vs torch decode backend (C4 shape)")
    ap.add_argument("--fusion-sweep", action="store_true",
                    help="persistent kernel at fusion_groups 1/2/4/7/14/28, batch 1 and 8")
    ap.add_argument("--pmc-collect", action="store_true",
                    help="rocprofv3 FETCH_SIZE/WRITE_SIZE passes (child processes) -> gpurun_out/pmc_traffic.json")
    ap.add_argument("--pmc-batches", default="",
                    help="with --only-kernel: run the timed loop at each of these batch sizes (PMC passes)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode step runs TP=1 on a single MI355X; "
              "multi-GPU data parallelism is independent replicas of this step. Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if args.pmc_collect:
        # (children do the GPU work; this process never touches the device)
        out = os.path.join(ROOT, "gpurun_out", "pmc_traffic.json")
        os.makedirs(os.path.dirname(out), exist_ok=True)
        print(json.dumps(pmc_collect(out)))
        return
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.engine:
        print(json.dumps({"metric": "engine decode step wall time and decode tok/s", "n_gpus": 1,
                          "data": "synthetic (random-init bf16 weights seed 0, random prompts)",
                          "engine": [engine_runs(1, 16, 128), engine_runs(8, 512, 128)]}))
        return
    if args.workload != "c3" or args.fusion_sweep:
        res = {"metric": "device us/decode-step & tok/s at batch 1-8 vs 1.19GB HBM weight floor", "unit": "us/step",
               "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "dtype": "bf16",
               "data": "synthetic (random-init bf16 weights seed 0, random token ids)"}
        if args.fusion_sweep:
            res["fusion_sweep"] = fusion_sweep(args.steps, args.warmup)
        else:
            res["workload"] = args.workload
            res["modes"] = long_context_runs(args.workload, args.steps, args.warmup)
        print(json.dumps(res))
        return
    _, _, _, dec = build_decoder(num_blocks=8 * 8 + 8, variant=args.variant, attn_splits=args.attn_splits)
    if args.only_kernel and args.pmc_batches:
        for b in (int(x) for x in args.pmc_batches.split(",")):
            el, _, _ = time_decode(dec, b, [args.start_ctx] * b, args.steps, args.warmup, args.mode)
            print(json.dumps({"batch": b, "ms_per_step": el * 1e3 / args.steps}), flush=True)
        dec.close()
        return
    start = [args.start_ctx] * args.batch
    elapsed, durs, contexts = time_decode(dec, args.batch, start, args.steps, args.warmup, args.mode,
                                          per_launch_events=True)
    if args.only_kernel:
        print(json.dumps({"ms_per_step": elapsed * 1e3 / args.steps}))
        return
    ms_per_step = elapsed * 1e3 / args.steps
    avg_launch_ms = sum(durs) / len(durs)
    bytes_per_launch = sum(step_bytes(c) for c in contexts) / len(contexts)
    achieved = bytes_per_launch / (avg_launch_ms * 1e-3) / 1e9
    if args.mode == "persistent":
        kernel = f"{PERSISTENT_KERNELS[args.variant]}<{args.batch}> (one launch per decode step)"
        traffic, traffic_src = measured_traffic(f"{PERSISTENT_KERNELS[args.variant]}<{args.batch}>")
    else:
        kernel = f"all stage kernels of one step ({args.mode})"
        traffic, traffic_src = None, "per-op path: no single dominant kernel"
    result = {
        "metric": "device us/decode-step & tok/s at batch 1-8 vs 1.19GB HBM weight floor",
        "value": round(args.batch * args.steps / elapsed, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "weight_floor_us_at_8TBps": round(WEIGHT_BYTES / HBM_PEAK_GBPS / 1e3, 2),
        "x_floor": round(ms_per_step * 1e3 / (WEIGHT_BYTES / HBM_PEAK_GBPS / 1e3), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights seed 0, random start token)",
        "config": {"workload": "C3: Qwen3-0.6B geometry decode, batch %d, context 1->%d, greedy, "
                               "device-resident token feedback" % (args.batch, args.steps),
                   "model": "Qwen3-0.6B geometry (random init)", "global_batch": args.batch,
                   "seq_len": args.steps, "parallelism": "single GPU (tp1)", "launch": args.mode},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src, "kernel": kernel,
                     "bytes_per_launch": int(bytes_per_launch), "avg_launch_us": round(avg_launch_ms * 1e3, 2)},
    }
    if not args.no_sweep:
        progress("sweep: batch 1-8 short context")
        sweep = {}
        for mode in ("persistent", "graph"):
            for b in (1, 2, 4, 8):
                el, d2, ctxs = time_decode(dec, b, [0] * b, 32, 4, mode, per_launch_events=True)
                us = sum(d2) / len(d2) * 1e3
                sweep[f"{mode}_b{b}"] = {"us_per_step": round(us, 2), "tok_per_s": round(b / us * 1e6, 1),
                                         "GBps": round(sum(step_bytes(c) for c in ctxs) / len(ctxs) / us / 1e3, 1)}
        result["sweep"] = sweep
        # C5 (prompt lengths U[1024,1920], ragged tables): the same boundary at long context
        progress("sweep: C5 long contexts")
        result["sweep_long_c5"] = long_context_runs("c5", 32, 4, dec=dec)
        progress("sweep: C4")
        result["sweep_long_c4"] = long_context_runs("c4", 32, 4, dec=dec)
    if not args.no_cpu_baseline:
        progress("cpu baseline")
        result["cpu_baseline"] = cpu_baseline()
    dec.close()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
