"""CPU oracle of the checkpoint-compression hot path — TEST INFRASTRUCTURE ONLY.

ctypes view of oracle/libckr_oracle.so (a C++ restatement of the reference's
code, see ckr_oracle.cpp for the file:line each function follows).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
only as the checker or the timed CPU baseline; the product never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libckr_oracle.so")

HEADER_DTYPE = np.dtype([("final_state", "<u4"), ("byte_count", "<u4"), ("buf_offset", "<u4"), ("pad", "<u4")])
TABLE_DTYPE = np.dtype([("norm_freq", "<u4", 256), ("cum_freq", "<u4", 257), ("x_max", "<u4", 256),
                        ("decode_sym", "u1", 4096), ("decode_freq", "<u4", 4096), ("decode_cum", "<u4", 4096),
                        ("_pad", "u1", 60)])
assert TABLE_DTYPE.itemsize == 40000

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "libckr_oracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, u64, i32, u32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_uint32
        sig = {
            "oc_element_size": (i32, [i32]),
            "oc_sidecar_per_elem": (i32, [i32]),
            "oc_extract_mantissa": (i32, [vp, u64, i32, vp, vp]),
            "oc_byte_hist": (None, [vp, u64, vp]),
            "oc_extract_mantissa_mt": (i32, [vp, u64, i32, vp, vp, i32]),
            "oc_byte_hist_mt": (None, [vp, u64, vp, i32]),
            "oc_normalize_histogram": (u32, [vp, i32, vp]),
            "oc_num_units": (u64, [u64, u64]),
            "oc_encode": (u64, [vp, u64, vp, u64, vp, vp, vp, i32]),
            "oc_decode": (u64, [vp, vp, vp, vp, u64, u64, vp]),
            "oc_merge_sidecar": (None, [vp, vp, u64, i32, vp]),
            "oc_tensor_stats": (None, [vp, u64, i32, u32, vp, vp, vp, vp]),
            "oc_repair_bucket_count": (u64, [u64]),
            "oc_repair_build": (u32, [vp, u64, i32, u32, u32, vp, vp, vp, vp]),
            "oc_repair_apply": (u64, [vp, u64, i32, u32, vp, u32, vp]),
            "oc_repair_last_tied_rounds": (u32, []),
        }
        for k, (r, a) in sig.items():
            f = getattr(L, k)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data


ES = {0: 4, 1: 2, 2: 2, 3: 1, 4: 4}
SPE = {0: 2, 1: 1, 2: 1, 3: 0, 4: 0}


def as_bytes(arr):
    return np.ascontiguousarray(arr).view(np.uint8).reshape(-1)


def extract_mantissa(raw, n, dtype, n_threads=1):
    """(masked bytes, sidecar bytes) of n elements given as raw bytes."""
    es, spe = ES[dtype], SPE[dtype]
    raw = as_bytes(raw)
    masked = np.empty(n * es, np.uint8)
    side = np.empty(max(n * spe, 1), np.uint8)
    if n_threads > 1:
        got = lib().oc_extract_mantissa_mt(_p(raw), n, dtype, _p(masked), _p(side), n_threads)
    else:
        got = lib().oc_extract_mantissa(_p(raw), n, dtype, _p(masked), _p(side))
    if got == 0:
        return raw[: n * es].copy(), np.empty(0, np.uint8)
    return masked, side[: n * spe]


def byte_hist(data, n_threads=1):
    data = as_bytes(data)
    h = np.zeros(256, np.uint32)
    if n_threads > 1:
        lib().oc_byte_hist_mt(_p(data), data.size, _p(h), n_threads)
    else:
        lib().oc_byte_hist(_p(data), data.size, _p(h))
    return h


def normalize_histogram(hist, ensure_full_alphabet=False):
    """Returns (table record of TABLE_DTYPE, table sum)."""
    h = np.ascontiguousarray(np.asarray(hist, np.uint32))
    t = np.zeros(1, TABLE_DTYPE)
    s = lib().oc_normalize_histogram(_p(h), int(bool(ensure_full_alphabet)), _p(t))
    return t[0], int(s)


def num_units(n_b, unit):
    return int(lib().oc_num_units(n_b, unit))


def encode(masked, table, unit, n_threads=1):
    """Chunked encode of a masked byte stream: (data, headers, unit_offsets)."""
    masked = as_bytes(masked)
    nb = masked.size
    nu = num_units(nb, unit)
    t = np.zeros(1, TABLE_DTYPE)
    t[0] = table
    out = np.zeros(max(nb, 1), np.uint8)
    hdr = np.zeros(max(nu, 1) * 256, HEADER_DTYPE)
    off = np.zeros(nu + 1, np.uint64)
    total = lib().oc_encode(_p(masked), nb, _p(t), unit, _p(out), _p(hdr), _p(off), n_threads)
    return out[:total], hdr[: nu * 256], off


def decode(data, headers, unit_offsets, table, n_b, unit):
    """(masked bytes, bad lane count)."""
    t = np.zeros(1, TABLE_DTYPE)
    t[0] = table
    data = np.ascontiguousarray(data, np.uint8) if data.size else np.zeros(1, np.uint8)
    headers = np.ascontiguousarray(headers)
    off = np.ascontiguousarray(unit_offsets, np.uint64)
    out = np.zeros(max(n_b, 1), np.uint8)
    bad = lib().oc_decode(_p(data), _p(headers), _p(off), _p(t), n_b, unit, _p(out))
    return out[:n_b], int(bad)


def merge_sidecar(masked, sidecar, n, dtype):
    out = np.empty(n * ES[dtype], np.uint8)
    masked = as_bytes(masked)
    sidecar = as_bytes(sidecar) if sidecar.size else np.zeros(1, np.uint8)
    lib().oc_merge_sidecar(_p(masked), _p(sidecar), n, dtype, _p(out))
    return out


def tensor_stats(raw, n, dtype, bins=256):
    """Reference-order fp32 statistics + fp64 values: dict(histogram, moments, minmax, moments64)."""
    raw = as_bytes(raw) if n else np.zeros(4, np.uint8)
    nb = min(bins, 256)
    h = np.zeros(max(nb, 1), np.uint32)
    mom = np.zeros(4, np.float32)
    mm = np.zeros(2, np.float32)
    m64 = np.zeros(4, np.float64)
    lib().oc_tensor_stats(_p(raw), n, dtype, bins, _p(h), _p(mom), _p(mm), _p(m64))
    return dict(histogram=h[:nb], moments=mom, minmax=mm, moments64=m64)


def compress_tensor(raw, n, dtype, unit, ensure_full_alphabet=False, n_threads=1):
    """Whole reference compress path for one tensor: mask → histogram → table → encode
    (the encode's units spread over n_threads host threads; same bytes)."""
    masked, side = extract_mantissa(raw, n, dtype)
    table, tsum = normalize_histogram(byte_hist(masked), ensure_full_alphabet)
    data, hdr, off = encode(masked, table, unit, n_threads)
    return dict(masked=masked, sidecar=side, table=table, table_sum=tsum, data=data, headers=hdr, unit_offsets=off)


# ---- prefix-mask repair (Re-Pair over masked words)
REPAIR_LAYOUT = {"float32": (4, 23), "float16": (2, 10), "fp16": (2, 10), "bfloat16": (2, 7), "bf16": (2, 7)}


def repair_bucket_count(n):
    return int(lib().oc_repair_bucket_count(n))


def repair_build(raw, n, storage_bytes, masked_bits, max_rules=50, want_seq=False):
    """dict(rules=[(replacement, lhs, rhs, freq)], out_len, max_pair, seq)."""
    raw = as_bytes(raw) if n else np.zeros(4, np.uint8)
    rules = np.zeros(max(max_rules, 1) * 4, np.uint64)
    out_len = np.zeros(1, np.uint64)
    mp = np.zeros(1, np.uint64)
    seq = np.zeros(max(n, 1), np.uint64) if want_seq else None
    nr = lib().oc_repair_build(_p(raw), n, storage_bytes, masked_bits, max_rules, _p(rules), _p(out_len),
                               _p(mp), _p(seq) if want_seq else None)
    r = dict(rules=[tuple(int(v) for v in rules[4 * i:4 * i + 4]) for i in range(nr)],
             out_len=int(out_len[0]), max_pair=int(mp[0]), tied_rounds=int(lib().oc_repair_last_tied_rounds()))
    if want_seq:
        r["seq"] = seq[: r["out_len"]]
    return r


def repair_apply(raw, n, storage_bytes, masked_bits, rules, want_seq=False):
    raw = as_bytes(raw) if n else np.zeros(4, np.uint8)
    rr = np.array([v for rule in rules for v in rule] or [0], np.uint64)
    seq = np.zeros(max(n, 1), np.uint64) if want_seq else None
    m = int(lib().oc_repair_apply(_p(raw), n, storage_bytes, masked_bits, _p(rr), len(rules),
                                  _p(seq) if want_seq else None))
    return (m, seq[:m]) if want_seq else m


# ---- fingerprint weights and clusters (small n: plain Python)
def fingerprint_weights(fps):
    """TensorAnalyzer::compute_fingerprint_weights (src/TensorAnalyzer.cpp:322-380)."""
    fps = [[float(np.float32(v)) for v in row] for row in fps]
    n = len(fps)
    imp = []
    for d in range(5):
        m = sum(r[d] for r in fps)
        m2 = sum(r[d] * r[d] for r in fps)
        imp.append(m2 / n - (m / n) * (m / n) if n else 0.0)
    tot = sum(v + 1e-8 for v in imp)
    return [v / tot for v in imp]


def category_of(name):
    """build_knn_clusters name prefixes (src/TensorAnalyzer.cpp:452-457)."""
    for p, c in (("optimizer.exp_avg_sq::", "exp_avg_sq"), ("optimizer.exp_avg::", "exp_avg"),
                 ("master_weights::", "master_weights")):
        if name.startswith(p):
            return c
    return "model_state"


def cluster(names, fps):
    """TensorAnalyzer::build_knn_clusters (src/TensorAnalyzer.cpp:440-598):
    (cluster id per record or -1, thresholds per non-empty category)."""
    import math
    fps = [[float(np.float32(v)) for v in row] for row in fps]
    cats = {}
    for i, nm in enumerate(names):
        cats.setdefault(category_of(nm), []).append(i)
    out = [None] * len(names)
    thr_out = []
    nid = 0
    for cat in sorted(cats):
        idx = cats[cat]
        k = len(idx)
        mean = [sum(fps[i][d] for i in idx) / k for d in range(5)]
        sd = []
        for d in range(5):
            v = sum((fps[i][d] - mean[d]) ** 2 for i in idx) / k
            sd.append(1.0 if v < 1e-30 else math.sqrt(v))

        def dist(a, b):
            return math.sqrt(sum(((fps[idx[a]][d] - fps[idx[b]][d]) / sd[d]) ** 2 for d in range(5)))
        alld = sorted(dist(a, b) for a in range(k) for b in range(a + 1, k))
        thr = alld[len(alld) // 4] if alld else 0.0
        thr_out.append(thr)
        parent, rank = list(range(k)), [0] * k

        def find(x):
            while parent[x] != x:
                parent[x] = parent[parent[x]]
                x = parent[x]
            return x

        for a in range(k):
            for b in range(a + 1, k):
                if dist(a, b) < thr:
                    ra, rb = find(a), find(b)
                    if ra == rb:
                        continue
                    if rank[ra] < rank[rb]:
                        ra, rb = rb, ra
                    parent[rb] = ra
                    if rank[ra] == rank[rb]:
                        rank[ra] += 1
        groups = {}
        for a in range(k):
            groups.setdefault(find(a), []).append(a)
        for root in sorted(groups):
            mem = groups[root]
            if len(mem) >= 2:
                for a in mem:
                    out[idx[a]] = nid
                nid += 1
            else:
                out[idx[mem[0]]] = -1
    return out, thr_out
