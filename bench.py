"""Decode benchmark of the device-resident token loop (one MI355X).

Workload (the configuration the headline metric is quoted on): Qwen2-0.5B shape, .qwb with Q4_0 layer
planes (dim 896, 24 layers, 14 query / 2 KV heads, FFN 4864, RoPE theta 1e6) and a 65536-row Q8_0 head
with seeded head_ids; seeded N(0, 0.02) random-init weights written by host/synth; 24-token seeded prompt,
greedy, batch 1.  A step is one decode position: the whole forward() plus the argmax on the device, one
hipGraph replay.  `value` = timed steps / wall time between two device-wide synchronizations.

The timed mode is the strict one (every float operation in the reference's order: logits and ids bitwise those
of qwen.c / runq.c built strict IEEE, checked over the same workload in the same run, `strict_vs_reference`);
the fast mode (tree sums) is timed too and reported as the sub-record "fast".  --fast swaps the two.

  python bench.py [--gpus 1] [--steps 128] [--warmup 8] [--config c1|c2|c3|c4|c5] [--no-cpu] [--no-counters]
                  [--no-c5] [--no-c4] [--fast] [--single-mode]
  python bench.py --traffic-from D --traffic-all     (every kernel kind's HBM bytes per launch from the passes in D)
  python bench.py --trace-summary T.csv              (a rocprofv3 kernel trace grouped by kernel and grid)
  python bench.py --floor                            (a plain streaming read of each layer GEMV's bytes per launch)
  The default run (c3) also measures the Qwen2-7B shape (c5) and the 512-token batched prefill of its own model
  (c4), and reports them as the sub-records "c5" and "c4".
  roofline.traffic (HBM bytes per launch of the dominant kernel) comes from two rocprofv3 --pmc passes that the
  run starts itself as child processes (FETCH_SIZE, then WRITE_SIZE, over `bench.py --counters`: a calibration
  copy of 1 GiB, then the prompt and 4 decode steps as eager launches, in the timed mode), or from earlier passes:
    python bench.py --traffic-from D ...      (D/fetch, D/write: rocprofv3 -d directories of the two passes)
  (c4: the 512-token prompt as one batched int8-MFMA prefill, timed over --steps repetitions, in both modes)
  The c3 run also reports "dropin": the reference's own qwen.c host built with -DFPGA against libmatvec_hip.so
  over the same workload (its tok/s and its FPGA_CHECK max abs diff, default and LLM_STRICT=1).

Also reported: per-kernel roofline (each kernel kind's device time inside the replayed step graph, from HIP
events around graph replays with and without that kind's launches, and its algorithmic bytes per launch);
the greedy workload in both modes against the reference's own qwen.c / runq.c built strict IEEE (ids, and every
position's logits: bitwise for the strict mode, the relative error and first divergence for the fast mode); and
the reference's OpenMP build (oracle/_ref/qwen_fast, -O3 -ffast-math) timed on this host over the same workload,
with this host's logical CPU count and model name."""
import argparse
import importlib.util
import json
import os
import re
import subprocess
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "local-llama-pynq-z2_amd")
PEAK_HBM = 8000.0  # GB/s, MI355X
METRIC = "decode tok/s + GEMV HBM GB/s (% of peak), Q4_0 Qwen2-0.5B shape, batch 1"
CONFIGS = {
    "c1": dict(fmt="bin", preset="c1", seed=1, prompt=8, new=240, ctx=0, ref="runq",
               metric="decode tok/s + GEMV HBM GB/s (% of peak), Q8_0 llama2.c 288/6L shape, batch 1",
               workload="llama2.c-style .bin decode (dim 288, 6 layers, 6 heads, FFN 768, vocab 32000, seq_len 256, "
                        "Q8_0 group 32 with fp32 scales): 8-token prompt, greedy, batch 1"),
    "c2": dict(fmt="bin", preset="c2", seed=2, prompt=8, new=512, ctx=0, ref="runq",
               metric="decode tok/s + GEMV HBM GB/s (% of peak), Q8_0 llama2.c 768/12L shape, batch 1",
               workload="llama2.c-style .bin decode (dim 768, 12 layers, 12 heads, FFN 2048, vocab 32000, seq_len "
                        "1024, Q8_0 group 32 with fp32 scales): 8-token prompt, greedy, batch 1"),
    "c3": dict(fmt="qwb", preset="c3", seed=3, prompt=24, new=128, ctx=1024, ref="qwen", metric=METRIC,
               workload="Qwen2-0.5B shape .qwb decode (dim 896, 24 layers, 14/2 heads, FFN 4864, Q4_0 layers, "
                        "Q8_0 65536-row head): 24-token prompt, 128 greedy tokens, batch 1"),
    "c4": dict(fmt="qwb", preset="c3", seed=3, prompt=512, new=64, ctx=1024, ref="qwen", metric=METRIC,
               workload="Qwen2-0.5B shape .qwb prefill (dim 896, 24 layers, 14/2 heads, FFN 4864, Q4_0 layers): "
                        "512-token prompt as int8 MFMA GEMMs + causal attention, then 64 greedy tokens, batch 1"),
    "c5": dict(fmt="qwb", preset="c5", seed=5, prompt=32, new=256, ctx=4096, ref="qwen",
               metric="decode tok/s + GEMV HBM GB/s (% of peak), Q4_0 Qwen2-7B shape, batch 1",
               workload="Qwen2-7B shape .qwb decode (dim 3584, 28 layers, 28/4 heads of 128, FFN 18944, Q4_0 "
                        "layers, Q8_0 152064-row head): 32-token prompt, 256 greedy tokens, KV cache 4096, batch 1"),
}


def load_pkg():
    spec = importlib.util.spec_from_file_location("llm_hip", os.path.join(PKG, "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def model_file(cfg):
    d = os.environ.get("BENCH_MODEL_DIR", "/tmp/llm_hip_bench")
    os.makedirs(d, exist_ok=True)
    path = os.path.join(d, f"{cfg['preset']}_s{cfg['seed']}.{cfg['fmt']}")
    if not os.path.exists(path):
        t = time.time()
        subprocess.run([os.path.join(PKG, "host", "synth"), cfg["fmt"], path + ".tmp", cfg["preset"], str(cfg["seed"])],
                       check=True, capture_output=True)
        os.replace(path + ".tmp", path)
        log(f"wrote {path} ({os.path.getsize(path) / 2**20:.0f} MiB) in {time.time() - t:.1f} s")
    return path


def head_ids_of(path):
    with open(path, "rb") as f:
        b = f.read(256)
    dim, hid, L, nh, nkv, vocab, head_k = np.frombuffer(b, np.int32, 7, 8)
    kv = dim // nh * nkv
    pad = lambda n: (n + 63) & ~63
    off = 256 + pad(4 * dim) * 3 * L + pad(4 * kv) * 2 * L + pad(4 * dim)
    return np.fromfile(path, np.int32, int(head_k), offset=off)


def ref_args(cfg, path, prompt, n_new):
    """command-line of the reference host for the workload: qwen.c counts -n in new tokens, runq.c in
    positions (prompt included, runq.c:1200)"""
    ids = ",".join(map(str, prompt))
    if cfg["ref"] == "qwen":
        return [path, "--ids", ids, "-t", "0", "-n", str(n_new), "-c", str(cfg["ctx"])]
    return [path, "--ids", ids, "-t", "0", "-n", str(len(prompt) - 1 + n_new)]


def host_cpu():
    """(logical CPUs of this host, lscpu model name)"""
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        m = re.search(r"Model name:\s*(.+)", out)
        model = m.group(1).strip() if m else None
    except (OSError, subprocess.SubprocessError):
        pass
    return os.cpu_count(), model


def omp_threads():
    """OpenMP threads for the reference's CPU runs: this host's OMP_NUM_THREADS when set (the CPU share a GPU
    job gets on a shared host), else every logical CPU"""
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def cpu_baseline(cfg, path, prompt, n_new):
    """the reference's qwen.c / runq.c (OpenMP build) on this host over the workload: the prompt and n_new greedy
    tokens, decode rate in qwen.c's definition"""
    exe = os.path.join(REPO, "oracle", "_ref", "qwen_fast" if cfg["ref"] == "qwen" else "runq_ids_fast")
    if not os.path.exists(exe):
        return None
    threads = omp_threads()
    env = dict(os.environ, OMP_NUM_THREADS=str(threads))
    t = time.time()
    r = subprocess.run([exe] + ref_args(cfg, path, prompt, n_new), capture_output=True, text=True, env=env, timeout=900)
    wall = time.time() - t
    m = re.search(r"generated: (\d+) tokens, ([0-9.]+) tok/s", r.stderr)
    if r.returncode != 0 or not m:
        log(f"cpu baseline failed: {r.stderr[-400:]}")
        return None
    src = "qwen.c" if cfg["ref"] == "qwen" else "runq.c"
    nproc, model = host_cpu()
    return {"value": float(m.group(2)), "unit": "tok/s", "cores": threads, "kind": "reference",
            "nproc": nproc, "cpu_model": model,
            "sample": f"{src} (OpenMP, {threads} threads = this host's OMP_NUM_THREADS, -O3 -ffast-math "
                      f"-march=x86-64-v3) on the same .{cfg['fmt']}: {len(prompt)}-token prompt + {int(m.group(1))} "
                      f"greedy tokens, decode rate in qwen.c's definition ({wall:.1f} s wall)"}


def reference_run(cfg, path, prompt, n_new, n_logits):
    """the reference's qwen.c / runq.c built strict IEEE (oracle/_ref/qwen, runq_ids) over the workload: its
    greedy ids and its --logits dump of every position"""
    exe = os.path.join(REPO, "oracle", "_ref", "qwen" if cfg["ref"] == "qwen" else "runq_ids")
    if not os.path.exists(exe):
        return None
    dump = os.path.join(os.environ.get("BENCH_MODEL_DIR", "/tmp/llm_hip_bench"), "ref.logits")
    r = subprocess.run([exe] + ref_args(cfg, path, prompt, n_new) + ["--logits", dump], capture_output=True, text=True,
                       timeout=900, env=dict(os.environ, OMP_NUM_THREADS=str(omp_threads())))
    if r.returncode != 0:
        log(f"reference run failed: {r.stderr[-400:]}")
        return None
    ids = [int(v) for v in r.stdout.strip().split(",") if v]
    return ids, np.fromfile(dump, np.float32).reshape(-1, n_logits)


def dropin_record(cfg, path, prompt, n_new, ref, n_logits):
    """the reference's own qwen.c host built unmodified with -DFPGA against libmatvec_hip.so (oracle/_ref/qwen-hip:
    every matmul() through fpga_matvec4, the rest of forward() and the sampler on the host cores) over the
    workload: its decode rate in qwen.c's definition, and its FPGA_CHECK line (every matmul also on the CPU,
    qwen.c:103-112) over 8 greedy tokens in the default mode and with LLM_STRICT=1 (groups added in the
    reference's order: the logits of every position then bitwise those of the strict CPU build)"""
    exe = os.path.join(REPO, "oracle", "_ref", "qwen-hip")
    if cfg["ref"] != "qwen" or not os.path.exists(exe):
        return None
    base = ref_args(cfg, path, prompt, n_new)

    def run(n, **env):
        args = base[:]
        args[args.index("-n") + 1] = str(n)
        dump = os.path.join(os.environ.get("BENCH_MODEL_DIR", "/tmp/llm_hip_bench"), "dropin.logits")
        r = subprocess.run([exe] + args + ["--logits", dump], capture_output=True, text=True, timeout=900,
                           env=dict(os.environ, OMP_NUM_THREADS=str(omp_threads()), **env))
        if r.returncode != 0:
            log(f"drop-in run failed: {r.stderr[-400:]}")
            return None
        rate = re.search(r"generated: (\d+) tokens, ([0-9.]+) tok/s", r.stderr)
        chk = re.search(r"FPGA_CHECK: (\d+) matmuls, max abs diff ([-0-9.e+na]+), max rel diff ([-0-9.e+na]+)",
                        r.stderr)
        ids = [int(v) for v in r.stdout.strip().split(",") if v]
        return {"ids": ids, "rate": float(rate.group(2)) if rate else None, "tokens": int(rate.group(1)) if rate else 0,
                "check": (int(chk.group(1)), float(chk.group(2)), float(chk.group(3))) if chk else None,
                "logits": np.fromfile(dump, np.float32).reshape(-1, n_logits)}

    timed = run(n_new)
    timed_strict = run(n_new, LLM_STRICT="1")
    fast = run(8, FPGA_CHECK="1")
    strict = run(8, FPGA_CHECK="1", LLM_STRICT="1")
    if not (timed and timed_strict and fast and strict):
        return None
    rec = {"value": timed["rate"], "unit": "tok/s", "tokens": timed["tokens"],
           "host": f"qwen.c -DFPGA (unmodified, strict IEEE build, OpenMP {omp_threads()} threads) + libmatvec_hip.so",
           "ids_equal_reference": bool(ref) and timed["ids"] == ref[0][:len(timed["ids"])],
           "fpga_check": {"matmuls": fast["check"][0], "max_abs_diff": fast["check"][1],
                          "max_rel_diff": fast["check"][2], "tokens": 8} if fast["check"] else None,
           "strict": {"value": timed_strict["rate"], "unit": "tok/s",
                      "ids_equal_reference": bool(ref) and timed_strict["ids"] == ref[0][:len(timed_strict["ids"])],
                      "fpga_check_matmuls": strict["check"][0] if strict["check"] else None,
                      "fpga_check_max_abs_diff": strict["check"][1] if strict["check"] else None,
                      "positions": int(len(strict["logits"])),
                      "bitwise_identical_logits": bool(ref) and len(ref[1]) >= len(strict["logits"]) and
                      bool(np.array_equal(strict["logits"], ref[1][:len(strict["logits"])]))},
           "reference_published": {"fpga_tok_s": 3.7, "fpga_check_max_abs_diff": 2.4e-4,
                                   "source": "the reference README: Qwen2.5-Coder-0.5B 4-bit on the PYNQ-Z2 overlay"}}
    log(f"drop-in (qwen.c -DFPGA on libmatvec_hip.so): {rec['value']} tok/s, FPGA_CHECK max abs diff "
        f"{rec['fpga_check'] and rec['fpga_check']['max_abs_diff']} (strict: {timed_strict['rate']} tok/s, "
        f"{rec['strict']['fpga_check_max_abs_diff']}, bitwise {rec['strict']['bitwise_identical_logits']})")
    return rec


def fast_parity(ref, prompt, ids_gpu, logits_gpu):
    """the fast mode's greedy ids and logits against the reference run; a divergence is reported with the
    reference's top-2 logit gap"""
    ids_ref, lg_ref = ref
    n = min(len(ids_ref), len(ids_gpu))
    div = next((i for i in range(n) if ids_ref[i] != ids_gpu[i]), None)
    rows = min(len(lg_ref), len(logits_gpu))
    upto = rows if div is None else len(prompt) + div  # positions on the shared token path
    errs = [float(np.abs(logits_gpu[p] - lg_ref[p]).max() / np.abs(lg_ref[p]).max()) for p in range(upto)]
    out = {"mode": "fast (tree sums)", "reference": "strict IEEE build", "tokens_compared": n,
           "identical": div is None, "first_divergence": div,
           "logit_rel_err_max": max(errs) if errs else None,
           "logit_rel_err_median": float(np.median(errs)) if errs else None}
    if div is not None:
        row = lg_ref[len(prompt) - 1 + div]
        top = np.sort(row)[-2:]
        out["reference_top2_gap_rel"] = float((top[1] - top[0]) / np.abs(row).max())
    return out


def strict_parity(ref, ids_gpu, logits_gpu, tok_s):
    """the strict mode's greedy ids and logits against the reference run: bit for bit"""
    ids_ref, lg_ref = ref
    rows = min(len(lg_ref), len(logits_gpu))
    same = rows == len(lg_ref) == len(logits_gpu) and all(np.array_equal(logits_gpu[p], lg_ref[p]) for p in range(rows))
    return {"mode": "strict (reference order)", "reference": "strict IEEE build", "positions": int(len(lg_ref)),
            "tokens": len(ids_ref), "bitwise_identical_logits": bool(same), "identical_ids": list(ids_ref) == list(ids_gpu),
            "tok_s": round(tok_s, 1) if tok_s else None}


# HIP kernel of each step kernel kind (.qwb models: int4 layers, int8 head), as the start of the name rocprofv3
# gives it (the template arguments after these, stream depth and load policy, vary)
KERNEL_SYMBOL = {"qkv_gemv": "k_gemv<4, 32, 0, 1, 2,", "o_gemv": "k_gemv<4, 32, 0, 2, 1,",
                 "gateup_gemv": "k_gemv<4, 32, 0, 1, 3,", "down_gemv": "k_gemv<4, 32, 0, 0, 1,",
                 "head_gemv": "k_gemv<8, 32, 0, 1, 4,", "attention": "k_attention", "step_start": "k_step_start"}
CALIB_BYTES = 1 << 30  # the plain device copy that calibrates the byte counters (larger than any load copy)


def calib_copy():
    """a plain elementwise pass over CALIB_BYTES (reads them once, writes them once) for the counter scale"""
    import torch
    a = torch.empty(CALIB_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    torch.mul(a, 2.0, out=b)
    torch.cuda.synchronize()
    del a, b
    torch.cuda.empty_cache()


def pmc_per_dispatch(csv_path, counter):
    """{kernel name: [KiB per dispatch]} from a rocprofv3 --pmc counter_collection.csv"""
    import csv
    out = {}
    for r in csv.DictReader(open(csv_path)):
        if r["Counter_Name"] == counter:
            out.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return out


def traffic_from(pmc_dir, kind):
    """HBM bytes per launch of `kind` from two rocprofv3 --pmc passes over `bench.py --calib` (FETCH_SIZE in
    pmc_dir/fetch, WRITE_SIZE in pmc_dir/write), each scaled by what the counter reads for the calibration copy
    (CALIB_BYTES read and CALIB_BYTES written)"""
    import glob
    res = {}
    for sub, counter in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE")):
        files = glob.glob(os.path.join(pmc_dir, sub, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            return None
        per = pmc_per_dispatch(files[0], counter)
        copy = [v for k, vs in per.items() if "copy" in k.lower() or "elementwise" in k.lower() for v in vs]
        sym = KERNEL_SYMBOL.get(kind)
        vals = [v for k, vs in per.items() if sym and sym in k for v in vs]
        if not copy or not vals:
            return None
        factor = max(copy) * 1024.0 / CALIB_BYTES  # counter bytes per real byte
        res[sub] = sum(vals) / len(vals) * 1024.0 / factor
        res[sub + "_factor"] = factor
    return res


def code_sizes():
    """{kind: {kernel: bytes of machine code}} of the decode kernels in the built library, read from its gfx950
    code object with the ROCm LLVM tools.  FETCH_SIZE counts a launch's instruction fetches too: every kernel
    starts with invalidated L2 caches, so each of the 8 XCDs fetches the code its waves execute, up to 8 x these
    bytes per launch."""
    import subprocess
    import tempfile
    llvm = "/opt/rocm/llvm/bin"
    lib = os.path.join(PKG, "libmatvec_hip.so")
    with tempfile.TemporaryDirectory() as td:
        fat, co = os.path.join(td, "fatbin"), os.path.join(td, "gfx950.co")
        subprocess.run(["objcopy", "--dump-section", f".hip_fatbin={fat}", lib], check=True)
        subprocess.run([f"{llvm}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fat}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True)
        syms = subprocess.run([f"{llvm}/llvm-readelf", "-s", "--wide", "--demangle", co], check=True,
                              capture_output=True, text=True).stdout
    sizes = {}
    for line in syms.splitlines():
        f = line.split(None, 7)
        if len(f) == 8 and f[3] == "FUNC":
            sizes[f[7]] = int(f[2])
    return {kind: {k: v for k, v in sorted(sizes.items()) if sym in k} for kind, sym in KERNEL_SYMBOL.items()}


def trace_summary(csv_path):
    """a rocprofv3 --kernel-trace CSV grouped by (kernel, grid, workgroup): share of GPU time, calls, avg / median /
    min / max microseconds (the prefill GEMM shapes share one kernel name and differ by grid)"""
    import csv
    groups = {}
    for r in csv.DictReader(open(csv_path)):
        # rocprofv3 writes Grid_Size / Workgroup_Size, or per-axis columns (Grid_Size_X, ...), by version
        grid = r.get("Grid_Size") or "x".join(r.get(f"Grid_Size_{c}", "") for c in "XYZ").strip("x")
        wg = r.get("Workgroup_Size") or r.get("Workgroup_Size_X", "")
        key = (r["Kernel_Name"], grid, wg)
        groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    total = sum(sum(v) for v in groups.values())
    for (name, grid, wg), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        v.sort()
        print(f"{sum(v) / total * 100:6.2f}%  calls {len(v):6d}  avg {sum(v) / len(v):9.2f}  med {v[len(v) // 2]:9.2f}  "
              f"min {v[0]:9.2f}  max {v[-1]:9.2f}  grid {grid:>9} wg {wg:>5}  {name}")


def layer_macs(info):
    """multiply-accumulates of the layer matrices for one token (qkv, o, gate/up, down)"""
    kv = info.dim // info.n_heads * info.n_kv_heads
    return info.n_layers * info.dim * (info.dim + 2 * kv + info.dim + 3 * info.hidden_dim)


def prefill_bench(a, cfg, path, prompt, reps=None):
    """C4: the prompt as one batched prefill, timed over `reps` (else `steps`) repetitions in the timed mode
    (strict unless --fast) and in the other mode; int8 ops counted on the layer GEMMs.  Returns the record."""
    import torch
    P = load_pkg()
    m = P.Model(path, cfg["ctx"])
    reps = reps or a.steps or 5
    ops_per_token = 2.0 * layer_macs(m.info)
    rates = {}
    for strict in ((not a.fast), a.fast):
        m.set_strict(strict)
        m.prefill(prompt)  # warmup (and the activation buffers)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            m.prefill(prompt)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / reps
        rates[strict] = wall
        log(f"prefill of {len(prompt)} tokens ({'strict' if strict else 'fast'}): {wall * 1e3:.2f} ms -> "
            f"{len(prompt) / wall:.0f} tok/s, layer GEMMs {ops_per_token * len(prompt) / 1e9:.1f} G int8 ops = "
            f"{ops_per_token * len(prompt) / wall / 1e12:.1f} TOP/s over the whole prefill")
    m.set_strict(not a.fast)
    gen = m.generate(prompt, cfg["new"])
    log(f"then {len(gen['ids'])} greedy tokens, decode {gen['timing'].decode_ms:.1f} ms")
    m.close()
    PEAK_I8 = 5000.0  # TOP/s, dense int8 MFMA
    wall = rates[not a.fast]
    ops = ops_per_token * len(prompt)
    other = rates[a.fast]
    out = {
        "metric": "prefill tok/s (int8 MFMA), Q4_0 Qwen2-0.5B shape, 512-token prompt",
        "value": round(len(prompt) / wall, 1), "unit": "tok/s", "n_gpus": 1, "steps": reps, "warmup": 1,
        "ms_per_step": round(wall * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic: seeded N(0,0.02) random-init weights, seeded prompt ids",
        "config": {"workload": cfg["workload"], "prompt_tokens": len(prompt), "ctx": cfg["ctx"], "batch": 1,
                   "mode": "fast (tree sums)" if a.fast else "strict (reference order)"},
        "roofline": {"bound": "mfma", "achieved": round(ops / wall / 1e12, 2), "peak": PEAK_I8, "unit": "TFLOP/s",
                     "frac": round(ops / wall / 1e12 / PEAK_I8, 5), "traffic": None,
                     "note": "int8 ops of the layer GEMMs over the whole prefill time (every kernel included)"},
        ("strict" if a.fast else "fast"): {"value": round(len(prompt) / other, 1), "ms_per_step": round(other * 1e3, 4),
                                           "frac": round(ops / other / 1e12 / PEAK_I8, 5)},
    }
    return out


def prompt_for(cfg, path):
    if cfg["fmt"] == "qwb":
        hid = head_ids_of(path)
        return [int(v) for v in np.random.default_rng(cfg["seed"]).choice(hid, cfg["prompt"], replace=False)]
    # runq: seeded ids from [2, vocab) (1 is BOS, which stops the generation)
    with open(path, "rb") as f:
        vocab = int(abs(np.frombuffer(f.read(64), np.int32, 1, 8 + 5 * 4)[0]))
    return [int(v) for v in np.random.default_rng(cfg["seed"]).integers(2, vocab, cfg["prompt"])]


def counter_traffic(config, kind, strict=True):
    """roofline.traffic: HBM bytes per launch of `kind` from two rocprofv3 --pmc passes (FETCH_SIZE, then
    WRITE_SIZE) over `bench.py --counters` as child processes, each pass with its own time limit; None when
    rocprofv3 is absent or a pass fails.  The passes launch the step's kernels eagerly (a pass over replayed
    step graphs once ended in a segmentation fault inside the profiled process)."""
    import shutil
    prof = shutil.which("rocprofv3")
    if not prof:
        return None
    d = os.path.join(os.environ.get("BENCH_MODEL_DIR", "/tmp/llm_hip_bench"), f"pmc_{config}")
    shutil.rmtree(d, ignore_errors=True)
    env = dict(os.environ, TMPDIR="/tmp")
    for sub, counter in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE")):
        cmd = ["timeout", "-s", "KILL", "180", prof, "--pmc", counter, "--output-format", "csv", "-d",
               os.path.join(d, sub), "-o", sub, "--", sys.executable, "-u", os.path.abspath(__file__), "--counters",
               "--config", config, "--profile-steps", "4"] + ([] if strict else ["--fast"])
        log(f"counter pass {counter}")
        r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True)
        if r.returncode != 0:
            log(f"counter pass {counter} failed (status {r.returncode}): {r.stderr[-300:]}")
            return None
    return traffic_from(d, kind)


def time_mode(m, name, prompt, steps, warmup, profile_steps, strict, sample):
    """timed greedy (or sampled) decode steps and the per-kernel in-graph profile of one mode: the record's
    numbers (tok/s, roofline of the dominant kernel, every kernel kind's in-graph time, all GEMVs together)"""
    import torch
    m.set_strict(strict)
    mode = "strict (reference order)" if strict else "fast (tree sums)"
    decoding = "argmax"
    if sample:
        t_, p_, s_ = sample.split(",")
        m.set_sampler(float(t_), float(p_), int(s_))
        decoding = f"sampler temperature {float(t_)} top-p {float(p_)} seed {int(s_)}"
    # warmup: W steps after the prompt, then back to the prompt's end for the timed steps
    m.generate(prompt, 1)
    if warmup:
        m.decode_replay(warmup)
    m.generate(prompt, 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_ms = m.decode_replay(steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    tok_s = steps / wall
    log(f"[{name}] {mode}: timed {steps} decode steps: {wall * 1e3:.2f} ms wall, {ev_ms:.2f} ms by events -> "
        f"{tok_s:.1f} tok/s")
    # per-kernel roofline: each kernel kind's time inside the replayed step graph
    m.set_sampler(0.0)
    m.generate(prompt, 1)
    eager = {s["name"]: s for s in m.profile(profile_steps)}
    m.generate(prompt, 1)
    stats, step_ms = m.profile_graph(profile_steps, rounds=3)
    total = sum(s["total_ms"] for s in stats)
    log(f"[{name}] {mode}: in-graph kernel times over {profile_steps} replayed steps (median step "
        f"{step_ms * 1e3:.1f} us, sum of kinds {total / profile_steps * 1e3:.1f} us):")
    for s in sorted(stats, key=lambda s: -s["total_ms"]):
        avg = s["total_ms"] / s["launches"]
        e = eager.get(s["name"])
        e_us = f"{e['total_ms'] / e['launches'] * 1e3:8.2f}" if e else "     -  "
        log(f"  {s['name']:12s} {s['launches']:6d} launches  avg {avg * 1e3:8.2f} us (eager {e_us} us)"
            f"  {s['total_ms'] / total * 100:5.1f}%  {s['bytes_per_launch'] / 1e6:8.3f} MB"
            f"  {s['bytes_per_launch'] / (avg * 1e-3) / 1e9:8.1f} GB/s")
    dom = max(stats, key=lambda s: s["total_ms"])
    dom_avg_s = dom["total_ms"] / dom["launches"] * 1e-3
    achieved = dom["bytes_per_launch"] / dom_avg_s / 1e9
    gemv = [s for s in stats if s["name"].endswith("_gemv")]
    gemv_bytes = sum(s["bytes_per_launch"] * s["launches"] for s in gemv)
    gemv_s = sum(s["total_ms"] for s in gemv) * 1e-3
    return {
        "mode": mode, "decoding": decoding, "tok_s": tok_s, "wall": wall, "dom": dom,
        "roofline": {"bound": "hbm", "kernel": dom["name"], "achieved": round(achieved, 1), "peak": PEAK_HBM,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM, 4), "traffic": None,
                     "avg_launch_us": round(dom_avg_s * 1e6, 3), "bytes_per_launch": round(dom["bytes_per_launch"])},
        "gemv_all": {"achieved": round(gemv_bytes / gemv_s / 1e9, 1), "unit": "GB/s",
                     "frac": round(gemv_bytes / gemv_s / 1e9 / PEAK_HBM, 4),
                     "share_of_step": round(sum(s["total_ms"] for s in gemv) / total, 4)},
        "kernels_in_graph": {s["name"]: {"avg_us": round(s["total_ms"] / s["launches"] * 1e3, 3),
                                         "GB_s": round(s["bytes_per_launch"] / (s["total_ms"] / s["launches"] * 1e-3) / 1e9, 1)}
                             for s in stats},
    }


def measure(a, name, steps, warmup, profile_steps, cpu_tokens, counters, baseline_tokens=None):
    """one configuration: the timed mode (strict, the reference's order, unless --fast) and the other mode as a
    labelled sub-record, each with its decode rate and in-graph per-kernel roofline; both modes' greedy runs
    against the reference's strict build over cpu_tokens greedy tokens (strict: bitwise); the reference's
    OpenMP build timed on this host over baseline_tokens (default cpu_tokens)"""
    cfg = CONFIGS[name]
    path = model_file(cfg)
    prompt = prompt_for(cfg, path)
    P = load_pkg()
    t = time.time()
    m = P.Model(path, cfg["ctx"])
    log(f"[{name}] model resident in {time.time() - t:.1f} s: {m.info.weight_bytes / 2**20:.0f} MiB of tiled weights, "
        f"{m.info.gemv_bytes_per_token / 1e6:.2f} MB GEMV bytes per token")
    if len(prompt) + 1 + max(steps, warmup, profile_steps, cpu_tokens) >= m.info.ctx:
        raise SystemExit("steps do not fit the context")
    strict_main = not a.fast
    # greedy runs of the parity workload in both modes, with every position's logits
    runs = {}
    for st in (True, False):
        m.set_strict(st)
        g = m.generate(prompt, cpu_tokens, logits=True)
        runs[st] = ([int(v) for v in g["ids"]], g["logits"])
        log(f"[{name}] {'strict' if st else 'fast'} greedy run: {len(g['ids'])} tokens, device decode "
            f"{g['timing'].decode_ms:.1f} ms")
    main = time_mode(m, name, prompt, steps, warmup, profile_steps, strict_main, a.sample)
    other = None if a.single_mode else time_mode(m, name, prompt, min(steps, 64), warmup, profile_steps,
                                                 not strict_main, a.sample)
    n_logits = m.info.n_logits
    m.close()

    ref = None if a.no_cpu else reference_run(cfg, path, prompt, cpu_tokens, n_logits)
    traffic = None
    if a.traffic_from:
        traffic = traffic_from(a.traffic_from, main["dom"]["name"])
    elif counters:
        traffic = counter_traffic(name, main["dom"]["name"], strict_main)
    if traffic:
        log(f"[{name}] traffic of {main['dom']['name']}: {traffic['fetch'] / 1e6:.3f} MB fetched + "
            f"{traffic['write'] / 1e6:.3f} MB written per launch (counter factors {traffic['fetch_factor']:.3f} / "
            f"{traffic['write_factor']:.3f})")
        main["roofline"]["traffic"] = round(traffic["fetch"] + traffic["write"])
    cpu = None if a.no_cpu else cpu_baseline(cfg, path, prompt, baseline_tokens or cpu_tokens)
    dropin = None if a.no_cpu or name != "c3" else dropin_record(cfg, path, prompt, cpu_tokens, ref, n_logits)
    strict_rec = main if strict_main else other
    fast_rec = other if strict_main else main
    out = {
        "metric": cfg["metric"],
        "value": round(main["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(main["wall"] / steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: seeded N(0,0.02) random-init weights (" + ("Q4_0 layers, Q8_0 head" if cfg["fmt"] == "qwb"
                 else "Q8_0 with fp32 scales") + "), seeded prompt ids",
        "config": {"workload": cfg["workload"], "prompt_tokens": len(prompt), "decode_steps": steps,
                   "decoding": main["decoding"], "mode": main["mode"], "ctx": cfg["ctx"] or None, "batch": 1},
        "roofline": main["roofline"],
        "gemv_all": main["gemv_all"],
        "kernels_in_graph": main["kernels_in_graph"],
        "cpu_baseline": cpu,
        "strict_vs_reference": (strict_parity(ref, *runs[True], strict_rec["tok_s"] if strict_rec else None)
                                if ref else None),
    }
    if other is not None:
        sub = {k: other[k] for k in ("mode", "roofline", "gemv_all", "kernels_in_graph")}
        sub["value"] = round(other["tok_s"], 2)
        sub["ms_per_step"] = round(other["wall"] / min(steps, 64) * 1e3, 4)
        sub["steps"] = min(steps, 64)
        if ref and fast_rec is other:
            sub["greedy_vs_reference"] = fast_parity(ref, prompt, *runs[False])
        out["fast" if strict_main else "strict"] = sub
    if ref and not strict_main:
        out["greedy_vs_reference"] = fast_parity(ref, prompt, *runs[False])
    if dropin:
        out["dropin"] = dropin
    return out


FLOOR_SHAPES = {  # (dim, hidden, kv_dim, layers) of the Qwen2 shapes; every layer matrix Q4_0 (fp16 scales, groups of 32)
    "c3": (896, 4864, 128, 24),
    "c5": (3584, 18944, 512, 28),
}


def gemv_bytes(d, n, wbits=4, gs=32, s=2):
    """algorithmic bytes of one GEMV launch: weights, scales, int8 input and its scales, fp32 output"""
    return d * n * wbits // 8 + d * (n // gs) * s + n + (n // gs) * 4 + d * 4


def read_floor(a):
    """the floor of one launch: a plain streaming read of each layer GEMV's algorithmic bytes, one launch per
    layer over distinct buffers in a graph (so no launch finds its bytes in a cache), non-temporal loads as the
    decode GEMVs use at these sizes, over several grid sizes; against the GEMVs' in-graph times of a bench run"""
    P = load_pkg()
    out = {"metric": "plain-read floor per launch (us, GB/s, fraction of 8 TB/s)", "shapes": {}}
    for name, (dim, hid, kv, layers) in FLOOR_SHAPES.items():
        kinds = {"qkv_gemv": gemv_bytes(dim + 2 * kv, dim), "o_gemv": gemv_bytes(dim, dim),
                 "gateup_gemv": gemv_bytes(2 * hid, dim), "down_gemv": gemv_bytes(dim, hid)}
        rec = {}
        for kind, nbytes in kinds.items():
            grid = {}
            for blocks in (256, 512, 1024, 2048):
                us = P.read_floor(nbytes, layers, blocks, nt=True, reps=20)
                grid[blocks] = round(us, 3)
            best = min(grid.values())
            rec[kind] = {"bytes": nbytes, "us": best, "GB_s": round(nbytes / best / 1e3, 1),
                         "frac": round(nbytes / best / 1e3 / 8000.0, 4), "us_by_blocks": grid}
            log(f"[floor {name}] {kind:12s} {nbytes / 1e6:8.3f} MB: {best:7.2f} us per launch, "
                f"{nbytes / best / 1e3:7.1f} GB/s ({nbytes / best / 1e3 / 80:.1f}% of 8 TB/s); by blocks {grid}")
        out["shapes"][name] = rec
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    ap.add_argument("--profile-steps", type=int, default=32)
    ap.add_argument("--cpu-tokens", type=int, default=None,
                    help="greedy tokens of the parity and CPU-baseline runs (default: the workload's)")
    ap.add_argument("--no-cpu", action="store_true", help="no reference runs (parity lines, CPU baseline)")
    ap.add_argument("--no-counters", action="store_true", help="no rocprofv3 counter passes (roofline.traffic null)")
    ap.add_argument("--no-c5", action="store_true", help="no Qwen2-7B-shape sub-record in the default run")
    ap.add_argument("--no-c4", action="store_true", help="no 512-token prefill sub-record in the default run")
    ap.add_argument("--fast", action="store_true",
                    help="time the fast (tree-sum) mode as the record and the strict (reference-order) mode as its "
                         "sub-record, instead of the other way round")
    ap.add_argument("--single-mode", action="store_true",
                    help="time the record's mode only (no sub-record of the other mode)")
    ap.add_argument("--sample", default=None, metavar="T,P,SEED",
                    help="decode with the on-device sampler (temperature, top-p, seed) instead of the argmax")
    ap.add_argument("--calib", action="store_true", help="run the counter calibration copy first")
    ap.add_argument("--counters", action="store_true",
                    help="counter pass: the calibration copy, then the prompt and --profile-steps decode steps as "
                         "eager launches only (no graphs), no report")
    ap.add_argument("--traffic-from", default=None, help="directory with the FETCH_SIZE/WRITE_SIZE passes")
    ap.add_argument("--traffic-all", action="store_true",
                    help="with --traffic-from: print every kernel kind's HBM bytes per launch and stop")
    ap.add_argument("--floor", action="store_true",
                    help="the plain-read floor of each layer GEMV's bytes per launch (C3 and C5 shapes), and stop")
    ap.add_argument("--code-sizes", action="store_true",
                    help="print the machine-code bytes of each decode kernel kind in the built library, and stop")
    ap.add_argument("--trace-summary", default=None, metavar="CSV",
                    help="print a rocprofv3 kernel trace grouped by kernel and grid, and stop")
    a = ap.parse_args()
    if a.trace_summary:
        return trace_summary(a.trace_summary)
    if a.code_sizes:
        for kind, ks in code_sizes().items():
            for k, b in ks.items():
                print(f"{kind:12s} {b / 1e3:6.1f} KB of code, x 8 XCDs {8 * b / 1e6:6.3f} MB  {k}")
        return
    if a.traffic_from and a.traffic_all:
        for kind in KERNEL_SYMBOL:
            r = traffic_from(a.traffic_from, kind)
            if r:
                print(f"{kind:14s} fetched {r['fetch'] / 1e6:9.3f} MB  written {r['write'] / 1e6:8.3f} MB per launch "
                      f"(counter factors {r['fetch_factor']:.3f} / {r['write_factor']:.3f})")
        return
    if a.gpus != 1:
        print(f"bench.py runs on one GPU: the decode path has no multi-GPU form (asked for --gpus {a.gpus})",
              file=sys.stderr)
        sys.exit(2)
    cfg = CONFIGS[a.config]
    steps = a.steps or cfg["new"]

    import torch
    assert torch.cuda.is_available(), "bench.py needs the GPU"
    torch.cuda.init()
    if a.floor:
        return read_floor(a)
    if a.calib or a.counters:
        calib_copy()
    if a.counters:
        path = model_file(cfg)
        prompt = prompt_for(cfg, path)
        P = load_pkg()
        m = P.Model(path, cfg["ctx"])
        m.set_strict(not a.fast)
        for pos, t in enumerate(prompt):
            m.forward(t, pos)
        m.profile(a.profile_steps)
        m.close()
        log(f"counter pass: {len(prompt)} eager positions + {a.profile_steps} profiled steps")
        return
    if a.config == "c4":
        path = model_file(cfg)
        print(json.dumps(prefill_bench(a, cfg, path, prompt_for(cfg, path))), flush=True)
        return
    out = measure(a, a.config, steps, a.warmup, a.profile_steps, a.cpu_tokens or cfg["new"], not a.no_counters)
    if a.config == "c3" and not a.no_c5:
        # the 7B-shape configuration, whose GEMVs carry the HBM roofline target: a shorter record (parity over the
        # prompt and 64 greedy tokens, the CPU reference timed over 8)
        c5 = measure(a, "c5", 32, 4, 8, a.cpu_tokens or 64, False, baseline_tokens=8)
        for k in ("n_gpus", "higher_is_better", "scaling", "vs_baseline", "dtype", "data"):
            c5.pop(k, None)
        out["c5"] = c5
    if a.config == "c3" and not a.no_c4:
        # the batched prefill of a 512-token prompt on the same model (int8 MFMA GEMMs): a short record
        c4cfg = CONFIGS["c4"]
        p4 = model_file(c4cfg)
        c4 = prefill_bench(a, c4cfg, p4, prompt_for(c4cfg, p4), reps=10)
        for k in ("n_gpus", "higher_is_better", "scaling", "vs_baseline", "dtype", "data"):
            c4.pop(k, None)
        out["c4"] = c4
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
