#!/usr/bin/env python3
"""Benchmark of the checkpoint-compression hot path on one MI355X.

Workload: the Llama-3-8B ZeRO-3 rank-0-of-8 shard,
1,003,782,656 elements in each of four tensors — bf16 params ~N(0,0.02), fp32
master = the same values upcast, fp32 exp_avg ~N(0,1e-3), fp32 exp_avg_sq =
N(0,1e-3)^2 + 1e-12 — 14.05 GB resident in HBM, coded in 64 KiB units.

A step is one full compression of the shard: per tensor the masked byte
histogram, the host table, the chunked rANS encode with sidecar split and
packing (ckr_compress).  `value` = uncompressed shard bytes / encode time per
step.  Decode of the same shard is timed the same way right after and reported
beside it, with the compression ratios, a bit-exact round-trip check, the
dominant kernel's roofline, and the CPU oracle timed on a bounded sample.

Config 5 (the Llama-3-70B rank shard, 123.5 GB resident in HBM, 1 MiB units)
streams: per tensor the masked histogram and table of the whole tensor, then the
tensor's 8 GiB slices encoded with that table one after the other into reused
buffers (slices end on unit boundaries, and units are independent given the
table, so each slice's units are the whole-tensor encode's), each decoded into
a reused window; as for the resident configurations, the lane checks (a
decode that counts failing lanes) and the comparison with the source run
outside the timed regions.

After the timed steps, the drop-in path runs end to end once per repetition:
checkers_py.initialize_context / analyze_tensors / compress_and_save on a
stand-in engine over the resident shard, writing the rank's files (v4, same
unit size) to a temporary directory; `compress_and_save` reports its wall time
and `container_ratio` is the shard's bytes over the bytes of those files.
`analyze` times ckr_analyze on the shard (one call, one record per tensor) and
`repair` cfg2's per-tensor prefix-mask repair build and apply.

Usage: python bench.py [--steps K] [--warmup W] [--config 3] [--unit 65536]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "encode/decode GB/s on 1 MI355X (8B ZeRO-3 rank shard) + compression ratio"
HBM_PEAK_GBPS = 8000.0

# element counts of the benchmark configurations
LLAMA8B_RANK0_OF_8 = 8_030_261_248 // 8
LLAMA70B_RANK0_OF_8 = 70_553_706_496 // 8


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_shard(cfg, torch, dev, seed=0):
    """Synthetic tensors of the configuration, generated on the GPU (torch Philox)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    tensors = []
    if cfg == 1:
        n = 4096 * 4096
        tensors.append(("exp_avg", (torch.randn(n, generator=g, device=dev) * 1e-3).contiguous()))
    elif cfg in (3, 5):
        n = LLAMA8B_RANK0_OF_8 if cfg == 3 else LLAMA70B_RANK0_OF_8
        p = (torch.randn(n, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        tensors.append(("params_bf16", p))
        tensors.append(("master_weights", p.float()))
        tensors.append(("exp_avg", torch.randn(n, generator=g, device=dev) * 1e-3))
        x = torch.randn(n, generator=g, device=dev).mul_(1e-3)
        tensors.append(("exp_avg_sq", x.mul_(x).add_(1e-12)))
    elif cfg == 2:
        shapes = [("q_proj", 4096 * 4096), ("k_proj", 1024 * 4096), ("v_proj", 1024 * 4096),
                  ("o_proj", 4096 * 4096), ("gate_proj", 14336 * 4096), ("up_proj", 14336 * 4096),
                  ("down_proj", 4096 * 14336)]
        for name, n in shapes:
            tensors.append((name, (torch.randn(n, generator=g, device=dev) * 0.02).to(torch.bfloat16)))
        for name in ("input_layernorm", "post_attention_layernorm"):
            tensors.append((name, torch.ones(4096, dtype=torch.bfloat16, device=dev)))
    elif cfg == 4:
        n = 256 * 1024 * 1024
        x = torch.exp(torch.randn(n, generator=g, device=dev) * 5.0 - 12.0)
        idx = torch.randint(0, n, (n // 1000,), generator=g, device=dev)
        x[idx] = 0.0
        idx = torch.randint(0, n, (n // 10000,), generator=g, device=dev)
        x[idx] = torch.rand(idx.numel(), generator=g, device=dev) * 1e-39
        idx = torch.randint(0, n, (n // 100000,), generator=g, device=dev)
        x[idx] = torch.tensor([float("inf"), float("-inf"), float("nan")], device=dev)[
            torch.randint(0, 3, (idx.numel(),), generator=g, device=dev)]
        blk = 16 * 1024 * 1024
        x.view(torch.int32)[:blk] = torch.randint(-2**31, 2**31 - 1, (blk,), generator=g, device=dev,
                                                  dtype=torch.int32)
        tensors.append(("adversarial", x))
    torch.cuda.synchronize()
    return tensors


def measured_traffic(kernel, cfg):
    """HBM bytes per launch of `kernel` on config `cfg` from the committed counter
    summary profiles/traffic_<kernel>_cfg<cfg>.json (FETCH_SIZE + WRITE_SIZE runs,
    scaled by the same counters on a copy of known size), or (None, None)."""
    path = os.path.join(ROOT, "profiles", f"traffic_{kernel}_cfg{cfg}.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        d = json.load(f)
    return int(d["hbm_bytes_per_launch"]), os.path.relpath(path, ROOT)


def host_cpu():
    """(logical CPUs the host reports, CPUs this process may use, CPU model)."""
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = nproc
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return nproc, avail, model


def cpu_baseline(shard, ck, sample_bytes_per_tensor, unit, reps=5):
    """The CPU oracle (C++ restatement of the reference's path; the reference has
    no CPU build of it) on the same synthetic tensors: per tensor the mask/sidecar
    split, the byte histogram, the table and the rANS encode, on an in-memory
    sample, best of `reps` timings after one warm-up.  Threaded leg: every step
    on the threads this GPU's share of the host allows (16 on these boxes, which
    run one GPU per 16 host threads), split and histogram over element ranges,
    encode over units; single-thread leg: every step on one thread, on an eighth
    of the sample."""
    import oracle as oc
    import torch
    nproc, avail, model = host_cpu()
    threads = max(1, min(avail, 16))
    samples = []
    for name, t in shard:
        tag = ck.torch_tag(t.dtype)
        es = t.element_size()
        n = min(t.numel(), sample_bytes_per_tensor // es)
        samples.append((tag, es, n, t[:n].contiguous().view(-1).cpu().view(torch.uint8).numpy()))

    def one_pass(nthr, div):
        total = 0
        t0 = time.perf_counter()
        for tag, es, n, raw in samples:
            m = max(1, n // div)
            masked, _ = oc.extract_mantissa(raw[: m * es], m, tag, n_threads=nthr)
            table, _ = oc.normalize_histogram(oc.byte_hist(masked, n_threads=nthr))
            oc.encode(masked, table, unit, n_threads=nthr)
            total += m * es
        return total, time.perf_counter() - t0

    def best(nthr, div):
        one_pass(nthr, div)  # warm-up
        runs = [one_pass(nthr, div) for _ in range(reps)]
        total = runs[0][0]
        return total, min(r[1] for r in runs), [round(r[1], 4) for r in runs]

    tot, sec, all_t = best(threads, 1)
    tot1, sec1, all_t1 = best(1, 8)
    host = dict(nproc=nproc, usable_cpus=avail, model=model)
    return dict(value=round(tot / sec / 1e9, 4), unit="GB/s", cores=threads, kind="port",
                sample=f"first {sample_bytes_per_tensor >> 20} MiB of each of the {len(shard)} tensors "
                       f"({tot / 1e6:.0f} MB): oracle split, histogram, table and rANS encode, "
                       f"{threads} threads (OpenMP over element ranges and {unit}-byte units), best of {reps}",
                seconds=round(sec, 4), runs_s=all_t, host=host,
                single_thread=dict(value=round(tot1 / sec1 / 1e9, 4), unit="GB/s", cores=1,
                                   sample=f"first {(sample_bytes_per_tensor // 8) >> 20} MiB of each tensor "
                                          f"({tot1 / 1e6:.0f} MB), every step on one thread, best of {reps}",
                                   seconds=round(sec1, 4), runs_s=all_t1))


def sha256_tensors(shard, chunk=1 << 28):
    """SHA-256 of each tensor's bytes (the seeded inputs behind a number), hashed
    on the host in 256 MiB pieces, one thread per tensor."""
    import hashlib
    from concurrent.futures import ThreadPoolExecutor
    import torch

    def one(t):
        h = hashlib.sha256()
        b = t.reshape(-1).view(torch.uint8)
        for i in range(0, b.numel(), chunk):
            h.update(b[i:i + chunk].cpu().numpy())
        return h.hexdigest()

    with ThreadPoolExecutor(max_workers=min(len(shard), 8)) as ex:
        return dict(zip([n for n, _ in shard], ex.map(one, [t for _, t in shard])))


def analyze_cpu_baseline(shard, ck, sample_bytes_per_tensor=512 << 20, piece=64 << 20, reps=3):
    """The oracle's statistics pass (its fp32 reduction order follows the
    reference kernel's 256 threads) on a bounded sample: the first
    `sample_bytes_per_tensor` of each tensor cut into `piece`-byte ranges, the
    ranges spread over the threads this GPU's share of the host allows; best of
    `reps` after a warm-up."""
    from concurrent.futures import ThreadPoolExecutor
    import oracle as oc
    import torch
    nproc, avail, model = host_cpu()
    threads = max(1, min(avail, 16))
    jobs = []
    for _, t in shard:
        tag = ck.torch_tag(t.dtype)
        es = t.element_size()
        n = min(t.numel(), sample_bytes_per_tensor // es)
        raw = t[:n].contiguous().view(torch.uint8).cpu().numpy()
        step = piece // es
        for i in range(0, n, step):
            m = min(step, n - i)
            jobs.append((raw[i * es:(i + m) * es], m, tag))
    total = sum(j[0].size for j in jobs)

    def run():
        t0 = time.perf_counter()
        with ThreadPoolExecutor(max_workers=threads) as ex:
            list(ex.map(lambda j: oc.tensor_stats(j[0], j[1], j[2], 256), jobs))
        return time.perf_counter() - t0

    run()
    sec = min(run() for _ in range(reps))
    return dict(value=round(total / sec / 1e9, 4), unit="GB/s", cores=threads, kind="port",
                sample=f"first {sample_bytes_per_tensor >> 20} MiB of each of the {len(shard)} tensors "
                       f"({total / 1e6:.0f} MB) in {piece >> 20} MiB ranges: the oracle's two-pass statistics "
                       f"(min/max/sum, then 256-bin histogram and central moments), {threads} threads over the "
                       f"ranges, best of {reps}", seconds=round(sec, 4), host=dict(nproc=nproc, model=model))


def repair_cpu_baseline(shard, names=("k_proj", "v_proj", "input_layernorm", "post_attention_layernorm")):
    """The oracle's Re-Pair (the reference CLI's loop: one std::unordered_map of
    pair counts per round, one thread) on cfg2's smaller tensors, 50 rules each,
    as the reference's CLI runs it."""
    import oracle as oc
    import torch
    d = dict(shard)
    per, tot_t, tot_n = [], 0.0, 0
    for name in names:
        t = d[name]
        raw = t.view(torch.uint8).cpu().numpy()
        t0 = time.perf_counter()
        r = oc.repair_build(raw, t.numel(), 2, 7, 50)
        sec = time.perf_counter() - t0
        per.append(dict(tensor=name, elements=t.numel(), rules=len(r["rules"]), build_ms=round(sec * 1e3, 2)))
        tot_t += sec
        tot_n += t.numel()
    return dict(value=round(tot_n / tot_t / 1e6, 3), unit="M elements/s", cores=1, kind="port",
                sample=f"grammar builds of {', '.join(names)} ({tot_n} bf16 words, 50 rules, all 7 mantissa bits "
                       "masked), one thread", seconds=round(tot_t, 3), tensors=per)


def reference_layout_leg(shard, ck, torch, dev):
    """The reference's own stream layout (unit_bytes 0: one stream of 256 lanes
    per tensor, the .ansc v2 files byte for byte) on one cfg3 fp32 tensor:
    encode (histogram, table, the long-unit kernels' two passes) and decode,
    each timed once with HIP events after a warm-up on the first 64 MiB."""
    name, t = [x for x in shard if x[1].dtype == torch.float32][0]
    tag = ck.torch_tag(t.dtype)
    n = t.numel()
    w = t[: 16 << 20]
    ck.decode(ck.compress(w, tag, 0))
    torch.cuda.synchronize()
    e = ck.Encoder(n, tag, 0, device=dev)
    a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    a.record()
    r = e.compress(t)
    b.record()
    torch.cuda.synchronize()
    dst = torch.empty(n * 4, dtype=torch.uint8, device=dev)
    d = ck.Decoder(n, tag, 0, device=dev)
    b2 = torch.cuda.Event(enable_timing=True)
    b2.record()
    bad = d.decode(r.data, r.headers, r.unit_offsets, r.table, r.sidecar, dst)
    c.record()
    torch.cuda.synchronize()
    ok = bad == 0 and torch.equal(dst, t.view(torch.uint8))
    enc_ms, dec_ms = a.elapsed_time(b), b2.elapsed_time(c)
    nb = n * 4
    log(f"[bench] reference layout (one stream) {name}: encode {enc_ms:.1f} ms, decode {dec_ms:.1f} ms, ok={ok}")
    out = dict(tensor=name, elements=n, unit_bytes=0, encode_ms=round(enc_ms, 3), decode_ms=round(dec_ms, 3),
               encode_GBps=round(nb / enc_ms / 1e6, 3), decode_GBps=round(nb / dec_ms / 1e6, 3),
               ans_ratio=round(nb / r.total, 4), roundtrip_bit_exact=ok,
               note="one unit: 256 lanes, each coding n/256 symbols in order; one thread per lane chain "
                    "records its state every 1024 rows (lu_chain_kernel), then every segment is coded side "
                    "by side (lu_code_kernel); the decode follows one chain per lane (decode_long_kernel). "
                    "The reference's own encode kernel runs 256 threads, one per lane")
    del e, r, d, dst
    torch.cuda.empty_cache()
    return out


def time_resident(shard, ck, torch, dev, unit, steps, warmup, sequential=False):
    """Warm-up, then `steps` timed whole-shard encodes (ckr_compress_many) and
    decodes (ckr_decode_many) with the inputs resident in HBM; then the bit-exact
    round trip and lane checks.  Returns the measurements and the objects."""
    encs = [ck.Encoder(t.numel(), ck.torch_tag(t.dtype), unit, device=dev) for _, t in shard]
    decs = [ck.Decoder(t.numel(), ck.torch_tag(t.dtype), unit, device=dev) for _, t in shard]
    dsts = [torch.empty_like(t) for _, t in shard]

    def encode_all():
        # the shard's tensors in one call: each histogram overlaps the previous
        # tensor's encode (sequential: one ckr_compress per tensor)
        if sequential:
            return [e.compress(t) for e, (_, t) in zip(encs, shard)]
        return ck.compress_many(encs, [t for _, t in shard])

    def decode_all(results, check=False):
        # the shard's tensors in one ckr_decode_many call (tensors up to 256 MiB
        # decoded side by side; sequential: one ckr_decode per tensor)
        if sequential:
            return [d.decode(r.data, r.headers, r.unit_offsets, r.table, r.sidecar, dst, check=check)
                    for d, r, dst in zip(decs, results, dsts)]
        return ck.decode_many(decs, results, dsts, check=check)

    for i in range(warmup):
        res = encode_all()
        decode_all(res)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        res = encode_all()
    ev1.record()
    torch.cuda.synchronize()
    enc_wall = (time.perf_counter() - t0) / steps
    enc_ev = ev0.elapsed_time(ev1) / 1e3 / steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        decode_all(res)
    ev1.record()
    torch.cuda.synchronize()
    dec_wall = (time.perf_counter() - t0) / steps
    dec_ev = ev0.elapsed_time(ev1) / 1e3 / steps
    bads = decode_all(res, check=True)
    roundtrip = all(torch.equal(d.view(torch.uint8), t.view(torch.uint8)) for d, (_, t) in zip(dsts, shard))
    ok = roundtrip and all(b == 0 for b in bads)
    n_in = sum(t.numel() * t.element_size() for _, t in shard)
    C = sum(r.total for r in res)
    S = sum(r.sidecar.numel() if r.sidecar is not None else 0 for r in res)
    n_units = sum(e.n_units for e in encs)
    H = n_units * 256 * 16 + (n_units + len(encs)) * 8 + len(encs) * 2308
    B = n_in + S + C + H
    m = dict(input_bytes=n_in, encode_ms=round(enc_wall * 1e3, 4), decode_ms=round(dec_wall * 1e3, 4),
             encode_ms_events=round(enc_ev * 1e3, 4), decode_ms_events=round(dec_ev * 1e3, 4),
             encode_GBps=round(n_in / enc_wall / 1e9, 3), decode_GBps=round(n_in / dec_wall / 1e9, 3),
             encode_roofline_frac=round(B / enc_wall / 1e9 / HBM_PEAK_GBPS, 4),
             decode_roofline_frac=round(B / dec_wall / 1e9 / HBM_PEAK_GBPS, 4),
             compressed_bytes=C, sidecar_bytes=S, header_bytes=H, units=n_units,
             ans_ratio=round(n_in / C, 4), disk_ratio=round(n_in / (C + S), 4),
             device_ratio=round(n_in / (C + S + H), 4), roundtrip_bit_exact=ok)
    state = dict(encs=encs, decs=decs, dsts=dsts, res=res, encode_all=encode_all, decode_all=decode_all,
                 enc_wall=enc_wall, dec_wall=dec_wall, enc_ev=enc_ev, dec_ev=dec_ev, C=C, S=S, H=H, ok=ok)
    return m, state


WORKLOADS = {1: "cfg1 fp32 4096x4096 N(0,1e-3)", 2: "cfg2 llama3-8b decoder layer bf16",
             3: "cfg3 llama3-8b zero3 rank0-of-8 shard (bf16 params, fp32 master, exp_avg, exp_avg_sq)",
             4: "cfg4 adversarial fp32 256M", 5: "cfg5 llama3-70b zero3 rank0-of-8 shard"}


def config_leg(cfg, ck, torch, dev, unit, steps, warmup):
    """One of the other resident configurations, measured as the headline is
    (encode and decode of the whole shard, round trip checked), with its
    inputs' SHA-256."""
    shard = make_shard(cfg, torch, dev)
    sha = sha256_tensors(shard)
    m, st = time_resident(shard, ck, torch, dev, unit, steps, warmup)
    m.update(workload=WORKLOADS[cfg], unit_bytes=unit, tensors=[n for n, _ in shard],
             elements_per_tensor=[t.numel() for _, t in shard], input_sha256=sha)
    log(f"[bench] cfg{cfg}: encode {m['encode_ms']:.3f} ms ({m['encode_roofline_frac']}), decode "
        f"{m['decode_ms']:.3f} ms ({m['decode_roofline_frac']}), ok={m['roundtrip_bit_exact']}")
    del st, shard
    torch.cuda.empty_cache()
    return m


class _ZeroParam:
    """A ZeRO-3 parameter as api.cpp reads it: requires_grad and ds_numel."""

    def __init__(self, n):
        self.requires_grad = True
        self.ds_numel = n


def save_leg(shard, torch, unit, reps=2):
    """End to end through the pybind drop-in: initialize_context on a stand-in
    engine holding the resident shard, analyze_tensors, then compress_and_save
    into a fresh directory (v4 states file with `unit`-byte units), timed on the
    wall clock from the call to its return with every file written.  cfg3's
    four tensors are one ZeRO-3 flat group (fp16 flat = params, fp32 flat =
    master, optimizer state = exp_avg, exp_avg_sq); other configs are plain
    parameters."""
    import shutil
    import tempfile
    import types

    import checkers_py
    named = dict(shard)
    if set(named) == {"params_bf16", "master_weights", "exp_avg", "exp_avg_sq"}:
        n = named["master_weights"].numel()
        p = _ZeroParam(n)
        opt = types.SimpleNamespace(
            fp16_partitioned_groups_flat=[named["params_bf16"]], fp32_partitioned_groups_flat=[named["master_weights"]],
            optimizer=types.SimpleNamespace(state={named["master_weights"]: {"exp_avg": named["exp_avg"],
                                                                            "exp_avg_sq": named["exp_avg_sq"]}}),
            grad_position={id(p): [0, 0, n]}, get_param_id=id)
        params = [("layers.flat", p)]
    else:
        opt, params = None, list(shard)
    eng = types.SimpleNamespace(module=types.SimpleNamespace(named_parameters=lambda: iter(params)),
                                optimizer=opt, global_rank=0)
    os.environ["CHECKERS_UNIT_BYTES"] = str(unit)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    checkers_py.initialize_context(eng)
    t_init = time.perf_counter() - t0
    t0 = time.perf_counter()
    checkers_py.analyze_tensors()
    t_an = time.perf_counter() - t0
    times, files = [], 0
    logf = tempfile.mktemp(prefix="ckr_bench_log_")
    os.environ["CHECKERS_LOG"] = logf   # the per-tensor lines of the reference's logger
    for r in range(reps):
        d = tempfile.mkdtemp(prefix="ckr_bench_")
        try:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            checkers_py.compress_and_save(d)
            times.append(time.perf_counter() - t0)
            files = sum(os.path.getsize(os.path.join(a, f)) for a, _, fs in os.walk(d) for f in fs)
        finally:
            shutil.rmtree(d, ignore_errors=True)
        log(f"[bench] compress_and_save {r + 1}/{reps}: {times[-1]:.3f} s, {files / 1e9:.3f} GB of files")
    del os.environ["CHECKERS_LOG"]
    per_tensor, timing = [], {}
    if os.path.exists(logf):
        lines = open(logf).read().splitlines()
        os.unlink(logf)
        # the last call's lines: its tensors, then its summary and [TIMING] lines
        last = max(i for i, ln in enumerate(lines) if "[summary]" in ln)
        first = max([i + 1 for i, ln in enumerate(lines[:last]) if ln.startswith("[TIMING]")] or [0])
        for ln in lines[first:last]:
            kv = dict(x.split("=", 1) for x in ln.split("] ", 2)[-1].split() if "=" in x)
            per_tensor.append({k: (v if k == "name" else float(v)) for k, v in kv.items()})
        for ln in lines[last + 1:]:
            if ln.startswith("[TIMING]"):
                k, v = ln.split()[1].split("=")
                timing[k] = float(v)
        # every call's totals: the first call's extra time against the later
        # ones, split into the writer's GPU work and the rest (files)
        calls = []
        for ln in lines:
            if ln.startswith("[TIMING]"):
                k, v = ln.split()[1].split("=")
                if k == "compress_and_save_total_ms":
                    calls.append({})
                if calls:
                    calls[-1][k] = float(v)
        timing["per_call"] = calls
    # a context over an engine with no parameters replaces this one: its arena,
    # the writer's buffers and its references to the shard go
    checkers_py.initialize_context(types.SimpleNamespace(
        module=types.SimpleNamespace(named_parameters=lambda: iter([])), optimizer=None, global_rank=0))
    return dict(seconds=[round(t, 4) for t in times], best_s=round(min(times), 4), file_bytes=files,
                initialize_context_s=round(t_init, 4), analyze_tensors_s=round(t_an, 4), unit_bytes=unit,
                records=4 if opt is not None else len(params), per_tensor=per_tensor, timing=timing)


def analyzer_leg(shard, ck, torch, steps):
    """ckr_analyze on the shard: one call with one record per tensor, timed with
    HIP events on the stream it runs on, then one profiled call for the
    per-kernel times.  Rooflines: B = n_in (the data read once, the bound of
    any statistics pass) and 2 n_in (what the two passes read: min/max and the
    sums, then histogram and central moments)."""
    an = ck.Analyzer([t for _, t in shard], [ck.torch_tag(t.dtype) for _, t in shard], bins=256)
    n_in = sum(t.numel() * t.element_size() for _, t in shard)
    for _ in range(2):
        an.run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        an.run()
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / steps
    ck.profile_begin()
    an.run()
    prof = ck.profile_end()
    kern = {k: dict(launches=c, total_ms=round(ms, 4)) for k, (c, ms) in prof.items()}
    passes = sum(prof[k][1] for k in ("stats_pass1_kernel", "stats_pass2_kernel") if k in prof) / 1e3
    for k in ("stats_pass1_kernel", "stats_pass2_kernel"):
        if k in prof:
            kern[k]["achieved_GBps"] = round(n_in / (prof[k][1] / 1e3) / 1e9, 2)
    log(f"[bench] analyze {t * 1e3:.3f} ms per call ({len(shard)} records)")
    return dict(ms=round(t * 1e3, 4), records=len(shard), input_bytes=n_in, GBps=round(n_in / t / 1e9, 2),
                roofline=dict(bound="hbm", kernel="stats_pass1_kernel + stats_pass2_kernel", peak=HBM_PEAK_GBPS,
                              unit="GB/s", achieved=round(n_in / t / 1e9, 2),
                              frac=round(n_in / t / 1e9 / HBM_PEAK_GBPS, 4),
                              achieved_two_pass=round(2 * n_in / t / 1e9, 2),
                              frac_two_pass=round(2 * n_in / t / 1e9 / HBM_PEAK_GBPS, 4),
                              passes_ms=round(passes * 1e3, 4)),
                kernels=kern)


def repair_leg(ck, torch, dev, cpu=True):
    """cfg2's prefix-mask repair, per tensor (the group is the tensor): the
    grammar build (at most 50 rounds, all 7 bf16 mantissa bits masked), then
    applying it again, each timed on the wall clock around its call (the build
    returns its rules to the host, so the call is complete when it returns).
    Roofline: each build round reads the tensor's words once, so the
    algorithmic bytes are B = n_in per round."""
    shard = make_shard(2, torch, dev)
    out, tot_b, tot_a, tot_bytes_rounds = [], 0.0, 0.0, 0
    n_max = max(t.numel() for _, t in shard)
    rp = ck.Repairer(n_max, ck.BF16, max_rules=50, device=dev)
    for name, t in shard:
        src = t.view(torch.uint8)
        w = rp.build(src)   # warm-up (first-use allocations, code paths, the rounds' graphs)
        rp.apply(src, w["rules"])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        r = rp.build(src)
        tb = time.perf_counter() - t0
        t0 = time.perf_counter()
        n_tok = rp.apply(src, r["rules"])
        ta = time.perf_counter() - t0
        assert n_tok == r["out_len"]
        rounds = len(r["rules"]) + (1 if len(r["rules"]) < 50 else 0)
        nb = t.numel() * t.element_size()
        tot_b += tb
        tot_a += ta
        tot_bytes_rounds += rounds * nb
        out.append(dict(tensor=name, elements=t.numel(), rules=len(r["rules"]), rounds=rounds, tokens=r["out_len"],
                        build_ms=round(tb * 1e3, 3), apply_ms=round(ta * 1e3, 3)))
    log(f"[bench] repair cfg2: build {tot_b * 1e3:.1f} ms, apply {tot_a * 1e3:.1f} ms over {len(shard)} tensors")
    ach = tot_bytes_rounds / tot_b / 1e9
    leg = dict(workload="cfg2 llama3-8b decoder layer bf16, group = each tensor, 50 rules", tensors=out,
               build_ms=round(tot_b * 1e3, 3), apply_ms=round(tot_a * 1e3, 3),
               roofline=dict(bound="hbm", kernel="repair build (all rounds)", unit="GB/s", peak=HBM_PEAK_GBPS,
                             achieved=round(ach, 2), frac=round(ach / HBM_PEAK_GBPS, 4),
                             algorithmic_bytes=tot_bytes_rounds),
               input_sha256=sha256_tensors(shard))
    if cpu:
        cb = repair_cpu_baseline(shard)
        names = {x["tensor"] for x in cb["tensors"]}
        g_ms = sum(x["build_ms"] for x in out if x["tensor"] in names)
        g_n = sum(x["elements"] for x in out if x["tensor"] in names)
        cb["gpu_same_sample"] = dict(value=round(g_n / (g_ms / 1e3) / 1e6, 3), unit="M elements/s",
                                     build_ms=round(g_ms, 3))
        leg["cpu_baseline"] = cb
        log(f"[bench] repair cpu {cb['value']} M elements/s (GPU {cb['gpu_same_sample']['value']} on the same tensors)")
    return leg


def copy_ceiling(torch, dev, nbytes=4 << 30, reps=10, batches=3):
    """HBM rates of plain streaming over a 4 GiB buffer, best of `batches`
    batches of `reps` launches each: a copy (read + written bytes per second) by
    torch's copy_ and by this build's 16-byte grid-stride probe
    (checkers_amd/libckr_probe.so, plain and non-temporal, 1024 to 16384
    workgroups), and a read-only pass.  The best copy is the practical ceiling
    for traffic that mixes reads and writes about evenly, as the encode and
    decode do."""
    import ctypes
    a = torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(7)
    b = torch.empty_like(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def best(fn):
        for _ in range(2):
            fn()
        runs = []
        for _ in range(batches):
            torch.cuda.synchronize()
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            runs.append(e0.elapsed_time(e1) / 1e3 / reps)
        return min(runs)

    rates = {"torch_copy": 2 * nbytes / best(lambda: b.copy_(a)) / 1e9}
    probe = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "checkers_amd", "libckr_probe.so"))
    probe.ckr_probe_hbm.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]
    st = torch.cuda.current_stream().cuda_stream

    def run(mode, blocks):
        if probe.ckr_probe_hbm(a.data_ptr(), b.data_ptr(), nbytes, mode, blocks, st):
            raise RuntimeError("ckr_probe_hbm failed")

    for mode, name in ((0, "probe_copy"), (1, "probe_copy_nt")):
        for blocks in (1024, 2048, 16384):
            rates[f"{name}_{blocks}"] = 2 * nbytes / best(lambda: run(mode, blocks)) / 1e9
    read = max(nbytes / best(lambda: run(2, blocks)) / 1e9 for blocks in (2048, 4096))
    del a, b
    top = max(rates, key=rates.get)
    return dict(GBps=round(rates[top], 2), best=top, read_GBps=round(read, 2),
                rates={k: round(v, 2) for k, v in rates.items()}, bytes_per_copy=2 * nbytes,
                kind="best device-to-device copy of a 4 GiB buffer (read + written bytes), best of 3 x 10 each")


def stream_bench(shard, ck, torch, dev, unit, steps, slice_bytes):
    """Config 5: histogram + table per tensor, then encode/decode slice by slice
    (reused buffers), every slice checked bit-exact against its source.
    Returns (encode seconds, decode seconds, C, S, H, n_units, ok)."""
    ev = lambda: torch.cuda.Event(enable_timing=True)
    enc_s = dec_s = 0.0
    C = S = H = units = 0
    ok = True
    for step in range(steps):
        C = S = H = units = 0
        for name, t in shard:
            tag = ck.torch_tag(t.dtype)
            es = t.element_size()
            n = t.numel()
            per = max(unit // es, (slice_bytes // unit) * (unit // es))  # elements per slice, whole units
            a, b = ev(), ev()
            a.record()
            # the masked histogram and the two live planes' (which size the
            # two-pass encoder's slots for the slices)
            hh = ck.byte_histogram(t, tag, planes=True).cpu().numpy().view(np.uint32)
            table, tsum = ck.build_table(hh[:256])
            planes = hh[256:] if ck.sidecar_bytes_per_elem(tag) else None
            b.record()
            torch.cuda.synchronize()
            enc_s += a.elapsed_time(b) / 1e3
            encs, decs = {}, {}
            window = None
            for s0 in range(0, n, per):
                m = min(per, n - s0)
                if m not in encs:
                    encs[m] = ck.Encoder(m, tag, unit, device=dev)
                    decs[m] = ck.Decoder(m, tag, unit, device=dev)
                if window is None:
                    window = torch.empty(per * es, dtype=torch.uint8, device=dev)
                src = t[s0:s0 + m]
                a, b, c = ev(), ev(), ev()
                a.record()
                r = encs[m].encode(src, table, planes=planes)
                b.record()
                decs[m].decode(r.data, r.headers, r.unit_offsets, r.table, r.sidecar, window, check=False)
                c.record()
                torch.cuda.synchronize()
                enc_s += a.elapsed_time(b) / 1e3
                dec_s += b.elapsed_time(c) / 1e3
                # as for the resident configurations, the lane checks in a decode
                # of their own outside the timed region
                bad = decs[m].decode(r.data, r.headers, r.unit_offsets, r.table, r.sidecar, window, check=True)
                ok = ok and bad == 0 and torch.equal(window[: m * es], src.view(torch.uint8))
                C += r.total
                S += m * ck.sidecar_bytes_per_elem(tag)
                units += encs[m].n_units
            del encs, decs, window
            log(f"[bench] {name}: {n * es / 1e9:.2f} GB streamed, ok={ok}")
        H = units * 256 * 16 + units * 8
    return enc_s / steps, dec_s / steps, C, S, H, units, ok


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--unit", type=int, default=65536)
    ap.add_argument("--cpu-sample-mib", type=int, default=1024)
    ap.add_argument("--slice-gib", type=int, default=8, help="config 5: slice size of the streamed encode/decode")
    ap.add_argument("--sequential", action="store_true", help="one ckr_compress and one ckr_decode per tensor, no overlap")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--no-save", action="store_true", help="skip the end-to-end compress_and_save leg")
    ap.add_argument("--no-analyze", action="store_true", help="skip the analyzer leg")
    ap.add_argument("--no-repair", action="store_true", help="skip cfg2's prefix-mask repair leg")
    ap.add_argument("--no-configs", action="store_true", help="skip the other configurations' legs (cfg1/2/4/5)")
    ap.add_argument("--no-cfg5", action="store_true", help="skip the cfg5 leg of the default run")
    ap.add_argument("--no-reference-layout", action="store_true", help="skip the one-stream (v2) leg")
    ap.add_argument("--no-sha", action="store_true", help="do not hash the inputs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 1 GiB device-to-device copy (known HBM traffic) for counter scaling")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (one ZeRO-3 rank's shard per GPU; "
              "ranks share nothing on this path). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import checkers_amd as ck
    ck.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    unit = args.unit if args.config != 5 else max(args.unit, 1 << 20)

    log(f"[bench] generating config {args.config} shard")
    shard = make_shard(args.config, torch, dev)
    n_in = sum(t.numel() * t.element_size() for _, t in shard)
    names, elems = [n for n, _ in shard], [t.numel() for _, t in shard]
    log(f"[bench] {len(shard)} tensors, {n_in / 1e9:.3f} GB; unit {unit}")
    sha = None if args.no_sha else sha256_tensors(shard)
    if args.config == 5:
        out = run_streamed(args, shard, ck, torch, dev, unit, n_in)
        out["config"]["input_sha256"] = sha
        print(json.dumps(out), flush=True)
        if not out["roundtrip_bit_exact"]:
            sys.exit(1)
        return

    if args.copy_calibration:  # 1 GiB read + 1 GiB written by one elementwise copy kernel
        a = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    m, st = time_resident(shard, ck, torch, dev, unit, args.steps, args.warmup, args.sequential)
    enc_wall, dec_wall, enc_ev, dec_ev = st["enc_wall"], st["dec_wall"], st["enc_ev"], st["dec_ev"]
    C, S, H, ok = st["C"], st["S"], st["H"], st["ok"]
    encs, encode_all, decode_all = st["encs"], st["encode_all"], st["decode_all"]
    log(f"[bench] encode {enc_wall * 1e3:.2f} ms/step wall, {enc_ev * 1e3:.2f} ms/step events")
    log(f"[bench] decode {dec_wall * 1e3:.2f} ms/step wall, {dec_ev * 1e3:.2f} ms/step events")
    log(f"[bench] roundtrip={ok} C={C / 1e9:.3f} GB S={S / 1e9:.3f} GB units={m['units']}")

    # ---- per-kernel profile of one encode + one decode
    kernels, roof = {}, None
    if not args.no_profile:
        ck.profile_begin()
        r2 = encode_all()
        decode_all(r2)
        prof = ck.profile_end()
        kernels = {k: dict(launches=c, total_ms=round(ms, 4), avg_ms=round(ms / c, 5)) for k, (c, ms) in prof.items()}
        # algorithmic bytes of each kernel over the whole shard (one encode, one
        # decode): what it must read and write at least once
        alg = {
            "encode_fast_kernel": n_in + S + C + H,   # read tensor; write sidecar, packed data, headers
            "encode_kernel": n_in + S + C,            # general path: read tensor, write sidecar + lane streams
            "masked_hist_kernel": n_in,               # read tensor
            "compact_kernel": 2 * C,                  # general path: read lane streams, write packed
            "decode_fast_kernel": C + S + H + n_in,   # read packed + sidecar + headers, write tensor
            "decode_kernel": C + S + n_in,            # general path
        }
        # only units taken by a kernel count for it: the general kernels run for
        # the few units the fast ones leave, so they are not the dominant kernel
        dom = max((k for k in alg if k in prof), key=lambda k: prof[k][1])
        ach = alg[dom] / (prof[dom][1] / 1e3) / 1e9
        traffic, tsrc = measured_traffic(dom, args.config)
        roof = dict(bound="hbm", kernel=dom, achieved=round(ach, 2), peak=HBM_PEAK_GBPS, unit="GB/s",
                    frac=round(ach / HBM_PEAK_GBPS, 4), traffic=traffic,
                    algorithmic_bytes=int(alg[dom]), launches=prof[dom][0],
                    avg_launch_ms=round(prof[dom][1] / prof[dom][0], 5))
        if tsrc:
            roof["traffic_source"] = tsrc
        if dom.startswith("encode") and not args.sequential:
            # the same kernel with nothing beside it (one ckr_compress per
            # tensor): compress_many runs the next tensor's histogram inside
            # the encoder's launches, which the figure above includes
            ck.profile_begin()
            for e, (_, t) in zip(encs, shard):
                e.compress(t)
            alone = ck.profile_end().get(dom)
            if alone:
                a_ach = alg[dom] / (alone[1] / 1e3) / 1e9
                roof["alone"] = dict(achieved=round(a_ach, 2), frac=round(a_ach / HBM_PEAK_GBPS, 4),
                                     avg_launch_ms=round(alone[1] / alone[0], 5))
        for k in alg:
            if k in prof:
                kernels[k]["achieved_GBps"] = round(alg[k] / (prof[k][1] / 1e3) / 1e9, 2)
        del r2

    # the encode reads the tensors twice (histogram, then the coder); its whole
    # HBM traffic and the decode's against a plain copy's rate
    copy = copy_ceiling(torch, dev)
    enc_traffic = 2 * n_in + S + C + H
    dec_traffic = C + S + H + n_in
    copy.update(encode_traffic_bytes=enc_traffic, decode_traffic_bytes=dec_traffic,
                encode_GBps=round(enc_traffic / enc_wall / 1e9, 2), decode_GBps=round(dec_traffic / dec_wall / 1e9, 2))
    copy.update(encode_frac=round(copy["encode_GBps"] / copy["GBps"], 4),
                decode_frac=round(copy["decode_GBps"] / copy["GBps"], 4))
    log(f"[bench] copy ceiling {copy['GBps']} GB/s; encode {copy['encode_frac']}, decode {copy['decode_frac']} of it")
    del st, encs, encode_all, decode_all
    torch.cuda.empty_cache()

    analyze = None
    if not args.no_analyze:
        analyze = analyzer_leg(shard, ck, torch, args.steps)
        if not args.no_cpu:
            analyze["cpu_baseline"] = analyze_cpu_baseline(shard, ck)
            log(f"[bench] analyze cpu {analyze['cpu_baseline']['value']} GB/s")
    repair = None if args.no_repair else repair_leg(ck, torch, dev, cpu=not args.no_cpu)

    reflayout = None
    if not args.no_reference_layout and args.config == 3:
        reflayout = reference_layout_leg(shard, ck, torch, dev)

    save = None
    if not args.no_save:
        save = save_leg(shard, torch, unit)
        save["GBps"] = round(n_in / save["best_s"] / 1e9, 3)

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline")
        cpu = cpu_baseline(shard, ck, args.cpu_sample_mib << 20, unit)
        log(f"[bench] cpu {cpu}")

    # the other configurations, each measured the same way (the headline's
    # shard is freed first; cfg5 streams 123.5 GB held in HBM)
    others = None
    if not args.no_configs and args.config == 3:
        del shard
        torch.cuda.empty_cache()
        others = {}
        for c in (1, 2, 4):
            others[f"cfg{c}"] = config_leg(c, ck, torch, dev, unit, args.steps, args.warmup)
        if not args.no_cfg5:
            sh5 = make_shard(5, torch, dev)
            n5 = sum(t.numel() * t.element_size() for _, t in sh5)
            sha5 = None if args.no_sha else sha256_tensors(sh5)
            o5 = run_streamed(argparse.Namespace(warmup=1, steps=1, slice_gib=args.slice_gib), sh5, ck, torch, dev,
                              1 << 20, n5)
            del sh5
            torch.cuda.empty_cache()
            keep = ("encode_ms", "decode_ms", "encode_GBps", "decode_GBps", "encode_roofline_frac",
                    "decode_roofline_frac", "compressed_bytes", "sidecar_bytes", "header_bytes", "ans_ratio",
                    "disk_ratio", "device_ratio", "roundtrip_bit_exact", "copy_ceiling")
            others["cfg5"] = {k: o5[k] for k in keep}
            others["cfg5"].update(workload=o5["config"]["workload"], unit_bytes=1 << 20, input_bytes=n5,
                                  steps=o5["steps"], input_sha256=sha5)
        ok = ok and all(v["roundtrip_bit_exact"] for v in others.values())

    out = {
        "metric": METRIC,
        "value": round(n_in / enc_wall / 1e9, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(enc_wall * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic: torch Philox on the GPU, seed 0, distributions of BASELINE.json configs",
        "config": {"workload": WORKLOADS[args.config], "elements_per_tensor": elems, "tensors": names,
                   "unit_bytes": unit, "input_bytes": n_in, "table_bits": 12, "lanes": 256, "input_sha256": sha},
        "encode_GBps": m["encode_GBps"],
        "decode_GBps": m["decode_GBps"],
        "encode_ms": round(enc_wall * 1e3, 3),
        "decode_ms": round(dec_wall * 1e3, 3),
        "encode_ms_events": round(enc_ev * 1e3, 3),
        "decode_ms_events": round(dec_ev * 1e3, 3),
        "encode_roofline_frac": m["encode_roofline_frac"],
        "decode_roofline_frac": m["decode_roofline_frac"],
        "compressed_bytes": C,
        "sidecar_bytes": S,
        "header_bytes": H,
        "ans_ratio": m["ans_ratio"],
        "disk_ratio": m["disk_ratio"],
        "device_ratio": m["device_ratio"],
        "container_ratio": round(n_in / save["file_bytes"], 4) if save else None,
        "roundtrip_bit_exact": ok,
        "compress_and_save": save,
        "analyze": analyze,
        "repair": repair,
        "reference_layout": reflayout,
        "configs": others,
        "roofline": roof,
        "copy_ceiling": copy,
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(out), flush=True)
    if not ok:
        sys.exit(1)


def run_streamed(args, shard, ck, torch, dev, unit, n_in):
    """Config 5 driver: warm-up on the first slice of the first tensor, then the
    streamed passes; one JSON line like the resident configs."""
    name0, t0 = shard[0]
    # a warm-up slice of at most 4 GiB: a larger one, taken as a tensor of its own,
    # could wrap the u32 histogram counts into a table that cannot be decoded
    w = min(t0.numel(), (min(args.slice_gib, 4) << 30) // t0.element_size())
    for _ in range(max(args.warmup, 1)):
        stream_bench([(name0, t0[:w])], ck, torch, dev, unit, 1, args.slice_gib << 30)
    steps = max(1, min(args.steps, 2))
    enc_s, dec_s, C, S, H, n_units, ok = stream_bench(shard, ck, torch, dev, unit, steps, args.slice_gib << 30)
    log(f"[bench] streamed: encode {enc_s * 1e3:.1f} ms, decode {dec_s * 1e3:.1f} ms, roundtrip={ok}")
    B = n_in + S + C + H
    # the streamed encode reads each slice three times (the tensor's histogram,
    # then the two passes of 1 MiB units)
    copy = copy_ceiling(torch, dev)
    enc_traffic, dec_traffic = 3 * n_in + S + C + H, B
    copy.update(encode_traffic_bytes=enc_traffic, decode_traffic_bytes=dec_traffic,
                encode_GBps=round(enc_traffic / enc_s / 1e9, 2), decode_GBps=round(dec_traffic / dec_s / 1e9, 2))
    copy.update(encode_frac=round(copy["encode_GBps"] / copy["GBps"], 4),
                decode_frac=round(copy["decode_GBps"] / copy["GBps"], 4))
    out = {
        "metric": METRIC, "value": round(n_in / enc_s / 1e9, 3), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": max(args.warmup, 1), "ms_per_step": round(enc_s * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic: torch Philox on the GPU, seed 0, distributions of BASELINE.json configs",
        "config": {"workload": "cfg5 llama3-70b zero3 rank0-of-8 shard, streamed in "
                               f"{args.slice_gib} GiB slices", "elements_per_tensor": [t.numel() for _, t in shard],
                   "tensors": [n for n, _ in shard], "unit_bytes": unit, "input_bytes": n_in,
                   "table_bits": 12, "lanes": 256},
        "encode_GBps": round(n_in / enc_s / 1e9, 3), "decode_GBps": round(n_in / dec_s / 1e9, 3),
        "encode_ms": round(enc_s * 1e3, 3), "decode_ms": round(dec_s * 1e3, 3),
        "encode_roofline_frac": round(B / enc_s / 1e9 / HBM_PEAK_GBPS, 4),
        "decode_roofline_frac": round(B / dec_s / 1e9 / HBM_PEAK_GBPS, 4),
        "compressed_bytes": C, "sidecar_bytes": S, "header_bytes": H,
        "ans_ratio": round(n_in / C, 4), "disk_ratio": round(n_in / (C + S), 4),
        "device_ratio": round(n_in / (C + S + H), 4), "container_ratio": None, "roundtrip_bit_exact": ok,
        "roofline": None, "copy_ceiling": copy, "cpu_baseline": None, "kernels": {},
    }
    return out


if __name__ == "__main__":
    main()
