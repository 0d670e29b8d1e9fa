"""Drop-in for the reference's Python module `checkers_py`
(src/python_bindings.cpp:17-35): initialize_context, analyze_tensors,
compress_and_save, over this library's C ABI.

    import checkers_amd.checkers_py as checkers_py     # instead of `import checkers_py`
    checkers_py.initialize_context(model_engine)       # api.cpp:899-1031
    checkers_py.analyze_tensors()                      # api.cpp:1033-1253
    checkers_py.compress_and_save(output_dir)          # api.cpp:1255-1299

The caller owns every tensor; the context keeps references to the tensors it
discovered (the reference's lifetime guard) and borrows their device memory.
Discovery follows api.cpp: the ZeRO-3 flat-group walk when the optimizer has
fp16/fp32_partitioned_groups_flat (:416-685), otherwise one record per named
parameter with local device storage (:852-885).  Record names, order and
dtype tags are the reference's, including its dtype parse, which tags
bfloat16 tensors as float16 (:887-893: "bfloat16" contains "float16").

Differences, all on inputs the reference mishandles: tensors that are not on a
GPU or not contiguous are skipped (the reference would hand their pointer to a
kernel), and tensors of a dtype without a tag are not written.
"""
import os
import sys

import checkers_amd as ck

_ctx = None


class _Record:
    __slots__ = ("name", "tensor", "tag", "n", "category")

    def __init__(self, name, tensor, tag, n, category):
        self.name, self.tensor, self.tag, self.n, self.category = name, tensor, tag, n, category


class _Context:
    def __init__(self, rank, bins):
        self.rank = rank
        self.bins = bins
        self.records = []
        self.skipped = 0
        self.cluster_of = None
        self.stats = None
        self.weights = None


def _parse_dtype(s):
    """parse_dtype (api.cpp:887-893): substring tests in this order."""
    if "float32" in s:
        return ck.F32
    if "float16" in s:
        return ck.F16
    if "bfloat16" in s:
        return ck.BF16
    if "int8" in s:
        return ck.I8
    return ck.UNKNOWN


def _extract_rank(engine, attr, env):
    """extract_rank (api.cpp:27-35)."""
    if hasattr(engine, attr):
        return int(getattr(engine, attr))
    v = os.environ.get(env)
    return int(v) if v is not None else -1


def _device_view(t):
    """The tensor if it can be borrowed (on a GPU, contiguous, non-empty)."""
    if t is None or not hasattr(t, "data_ptr") or not hasattr(t, "is_cuda"):
        return None
    if not t.is_cuda or not t.is_contiguous() or t.numel() == 0 or t.data_ptr() == 0:
        return None
    return t


def _add(ctx, name, t, category):
    t = _device_view(t)
    if t is None:
        return False
    ctx.records.append(_Record(name, t, _parse_dtype(str(t.dtype)), t.numel(), category))
    return True


def _group_rank(param, fallback):
    """extract_group_rank (api.cpp:690-710): rank inside the parameter's process group."""
    pg = getattr(param, "ds_process_group", None)
    if pg is None:
        return fallback
    try:
        import torch.distributed as dist
        if not dist.is_initialized():
            return fallback
        return dist.get_rank(group=pg)
    except Exception:
        return fallback


def _zero_partition(param, rank):
    """try_zero_partitioned_tensor (api.cpp:712-787): this rank's resident slice of ds_tensor."""
    h = getattr(param, "ds_tensor", None)
    if h is None:
        return None
    logical = int(getattr(param, "ds_numel", 0) or (h.numel() if hasattr(h, "numel") else 0))
    part = int(param.partition_numel()) if hasattr(param, "partition_numel") else int(getattr(h, "ds_numel", 0))
    if not logical or not part:
        return None
    r = _group_rank(param, rank)
    off = 0 if r < 0 else r * part
    if off >= logical:
        return None
    resident = min(part, logical - off)
    flat = h.reshape(-1)
    return flat[:resident] if resident <= flat.numel() else None


def _extract(param, rank):
    """extract_tensor (api.cpp:852-885): ds_tensor partition, the parameter, .data, _hp_mapping."""
    t = _zero_partition(param, rank)
    if _device_view(t) is not None:
        return t
    for cand in (getattr(param, "ds_tensor", None), param, getattr(param, "data", None),
                 getattr(getattr(param, "_hp_mapping", None), "hp_tensor", None)):
        if _device_view(cand) is not None:
            return cand
    return None


def _discover_zero3(ctx, opt, named, rank):
    """discover_zero3_flat_states (api.cpp:416-685)."""
    fp32 = list(getattr(opt, "fp32_partitioned_groups_flat", []) or [])
    fp16 = list(getattr(opt, "fp16_partitioned_groups_flat", []) or [])
    state = {}
    base = getattr(opt, "optimizer", None)
    if base is not None and isinstance(getattr(base, "state", None), dict):
        state = base.state
    if not fp32:
        return
    groups = [[] for _ in fp32]
    if hasattr(opt, "grad_position") and hasattr(opt, "get_param_id"):
        for pname, p in named:
            if not getattr(p, "requires_grad", False) or not hasattr(p, "ds_numel"):
                continue
            try:
                loc = opt.grad_position.get(opt.get_param_id(p), None)
                if loc is None:
                    continue
                g, foff, fn = (int(v) for v in list(loc)[:3])
                dsn = int(p.ds_numel)
                if g < len(fp32) and fn > 0 and dsn > 0:
                    groups[g].append((foff, pname, p, fn, dsn))
            except Exception:
                continue
        for gp in groups:
            gp.sort(key=lambda x: x[0])   # stable, as std::sort on distinct offsets
    for g, gp in enumerate(groups):
        if not gp:
            continue
        flat32 = fp32[g]
        size = int(flat32.numel())
        if size == 0:
            continue
        total = sum(x[4] for x in gp)
        lo, hi = rank * size, min((rank + 1) * size, total)
        flat16 = fp16[g] if g < len(fp16) else None
        ea = easq = None
        st = state.get(flat32) if state else None
        if isinstance(st, dict):
            ea, easq = st.get("exp_avg"), st.get("exp_avg_sq")
        pos = 0
        for foff, pname, p, fn, dsn in gp:
            s, e = pos, pos + dsn
            pos = e
            if e <= lo or s >= hi:
                ctx.skipped += 1
                continue
            got = 0
            if flat16 is not None:
                got += _add(ctx, pname, flat16.narrow(0, foff, fn), "model_state")
            else:
                t = _zero_partition(p, rank)
                got += _add(ctx, pname, t, "model_state")
            got += _add(ctx, "master_weights::" + pname, flat32.narrow(0, foff, fn), "master_weights")
            if ea is not None:
                got += _add(ctx, "optimizer.exp_avg::" + pname, ea.narrow(0, foff, fn), "exp_avg")
            if easq is not None:
                got += _add(ctx, "optimizer.exp_avg_sq::" + pname, easq.narrow(0, foff, fn), "exp_avg_sq")
            if not got:
                ctx.skipped += 1


def initialize_context(model_engine, optimizer=None, histogram_bins=256, background_threads=1):
    """Discover this rank's tensors (api.cpp:899-1031)."""
    global _ctx
    try:
        if histogram_bins == 0:
            raise RuntimeError("histogram_bins must be greater than zero")
        if background_threads == 0:
            raise RuntimeError("background_threads must be greater than zero")
        rank = _extract_rank(model_engine, "global_rank", "RANK")
        ctx = _Context(rank, int(histogram_bins))
        named = list(model_engine.module.named_parameters())
        opt = optimizer
        if opt is None:
            opt = getattr(model_engine, "optimizer", None)
        if opt is not None and hasattr(opt, "fp16_partitioned_groups_flat") and \
                hasattr(opt, "fp32_partitioned_groups_flat"):
            _discover_zero3(ctx, opt, named, rank)
        else:
            for name, p in named:
                t = _extract(p, rank)
                if t is None or not _add(ctx, name, t, "model_state"):
                    ctx.skipped += 1
        _ctx = ctx
    except Exception as e:
        raise RuntimeError("[checkers] Context initialization failed: " + str(e)) from e


def analyze_tensors():
    """Statistics, fingerprints, weights and clusters (api.cpp:1033-1253)."""
    try:
        if _ctx is None or not _ctx.records:
            return
        recs = _ctx.records
        # a record without a dtype tag keeps zero statistics (its stats buffers
        # are cleared and the kernel skips it, TensorAnalyzer.cpp:217-220)
        known = [i for i, r in enumerate(recs) if r.tag != ck.UNKNOWN]
        st = ck.analyze([recs[i].tensor for i in known], [recs[i].tag for i in known], bins=_ctx.bins)
        _ctx.stats = [None] * len(recs)
        fps = [[0.0] * 5 for _ in recs]
        for j, i in enumerate(known):
            _ctx.stats[i] = st[j]
            fps[i] = st[j]["fingerprint"]
        _ctx.weights = ck.fingerprint_weights(fps)
        _ctx.cluster_of, _ = ck.cluster([r.name for r in recs], fps)
    except Exception as e:
        print(f"[CHECKERS CRITICAL ERROR] {e}", file=sys.stderr, flush=True)
        raise


def compress_and_save(output_path, /, *, unit_bytes=0):
    """Write rank_<r>_states.ansc, mantissa/…mant and tables/…dict under
    output_path (api.cpp:1255-1299).  unit_bytes 0 writes the reference's v2
    states file; a unit size writes the chunked v3 layout."""
    try:
        if _ctx is None:
            raise RuntimeError("Context not initialized: call initialize_context first.")
        recs = [r for r in _ctx.records if r.tag != ck.UNKNOWN]
        cid = _ctx.cluster_of or [-1] * len(_ctx.records)
        ids = {id(r): c for r, c in zip(_ctx.records, cid)}
        ck.write_checkpoint(output_path, max(_ctx.rank, 0),
                            [(r.name, r.tensor, r.tag, ids[id(r)]) for r in recs], unit_bytes=unit_bytes)
    except Exception as e:
        print(f"[CHECKERS CRITICAL ERROR] compress_and_save: {e}", file=sys.stderr, flush=True)
        raise


def records():
    """(name, dtype tag, elements) of the discovered records, in record order."""
    return [] if _ctx is None else [(r.name, r.tag, r.n) for r in _ctx.records]
