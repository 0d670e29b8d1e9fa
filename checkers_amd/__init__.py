"""checkers_amd — MI355X (gfx950) checkpoint-compression hot path.

Python view of the C ABI in include/checkers_amd.h (libcheckers_amd.so, built
in-tree by checkers_amd/build.py).  Device buffers are torch tensors on the
current HIP device; torch is used only for device memory and streams.

Loading is strict: if the shared library is missing or fails to load, every
entry point raises.  There is no CPU fallback.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcheckers_amd.so")

# dtype tags: include/checkers/TensorResource.hpp:30-37 (reference)
F32, BF16, F16, I8, I32, UNKNOWN = 0, 1, 2, 3, 4, 255
M = 4096
L = 1 << 23
LANES = 256

CKR_OK, CKR_E_INVALID, CKR_E_HIP, CKR_E_CAPACITY, CKR_E_TABLE, CKR_E_CORRUPT = 0, -1, -2, -3, -4, -5

EXPORTED = [  # every symbol include/checkers_amd.h declares
    "ckr_last_error", "ckr_version", "ckr_element_size", "ckr_sidecar_bytes_per_elem",
    "ckr_extract_mantissa", "ckr_byte_histogram", "ckr_byte_histogram_raw", "ckr_byte_histogram_planes",
    "ckr_build_table", "ckr_build_table_ranked", "ckr_build_tables_device",
    "ckr_num_units", "ckr_encode_max_output_bytes", "ckr_encode_workspace_bytes", "ckr_encode",
    "ckr_encode_planes",
    "ckr_compress", "ckr_compress_many", "ckr_decode_workspace_bytes", "ckr_decode", "ckr_decode_many",
    "ckr_decode_noalloc", "ckr_analyze_workspace_bytes",
    "ckr_analyze", "ckr_profile_begin", "ckr_profile_end", "ckr_set_fast_paths",
    "ckr_repair_masked_bits", "ckr_repair_bucket_count", "ckr_repair_workspace_bytes",
    "ckr_repair_build", "ckr_repair_apply",
    "ckr_fingerprint_weights", "ckr_cluster", "ckr_ckpt_write", "ckr_ckpt_set_slice_bytes",
    "ckr_ckpt_slice_bytes", "ckr_ckpt_reserve", "ckr_ckpt_pool_bytes", "ckr_ckpt_release",
    "ckr_ckpt_open", "ckr_ckpt_count",
    "ckr_ckpt_info", "ckr_ckpt_restore", "ckr_ckpt_close",
    "ckr_arena_create", "ckr_arena_alloc", "ckr_arena_used", "ckr_arena_reset", "ckr_arena_destroy",
    "ckr_stats_slab_bytes", "ckr_carve_stats_slab", "ckr_analyze_device_records",
    "ckr_analyze_device_records_workspace_bytes", "ckr_make_contiguous",
]


class CkrError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{msg} (status {code})")
        self.code = code


class StreamHeader(ctypes.Structure):
    _fields_ = [("final_state", ctypes.c_uint32), ("byte_count", ctypes.c_uint32),
                ("buf_offset", ctypes.c_uint32), ("pad", ctypes.c_uint32)]


HEADER_DTYPE = np.dtype([("final_state", "<u4"), ("byte_count", "<u4"), ("buf_offset", "<u4"), ("pad", "<u4")])


class FreqTable(ctypes.Structure):
    """ckr_freq_table (40000 bytes, 64-byte aligned in C; see aligned_table())."""
    _fields_ = [("norm_freq", ctypes.c_uint32 * 256), ("cum_freq", ctypes.c_uint32 * 257),
                ("x_max", ctypes.c_uint32 * 256), ("decode_sym", ctypes.c_uint8 * 4096),
                ("decode_freq", ctypes.c_uint32 * 4096), ("decode_cum", ctypes.c_uint32 * 4096),
                ("_pad", ctypes.c_uint8 * 60)]


assert ctypes.sizeof(FreqTable) == 40000


class StatsRecord(ctypes.Structure):
    _fields_ = [("d_ptr", ctypes.c_void_p), ("num_elements", ctypes.c_uint64),
                ("histogram_bins", ctypes.c_uint32), ("data_type", ctypes.c_uint32),
                ("d_histogram", ctypes.c_void_p), ("d_raw_moments", ctypes.c_void_p),
                ("d_minmax", ctypes.c_void_p), ("d_fingerprint", ctypes.c_void_p)]


_TABLE_SPAN = 40000 + 64  # sizeof(ckr_freq_table) and room to align it


class _AlignedTable:
    """A FreqTable placed at a 64-byte aligned address (the C type is alignas(64)).
    The memory is not cleared: every library call that returns a table writes
    all of it.  buf/off: a slice of a buffer shared by several tables."""

    def __init__(self, buf=None, addr=None):
        self._buf = np.empty(_TABLE_SPAN, np.uint8) if buf is None else buf
        if addr is None:
            addr = self._buf.ctypes.data
        self.table = FreqTable.from_address((addr + 63) & ~63)

    @property
    def ptr(self):
        return ctypes.byref(self.table)

    @property
    def norm(self):
        return np.frombuffer(self.table.norm_freq, dtype=np.uint32).copy()

    @property
    def cum(self):
        return np.frombuffer(self.table.cum_freq, dtype=np.uint32).copy()

    def raw_bytes(self):
        return ctypes.string_at(ctypes.addressof(self.table), 40000 - 60)


def aligned_table():
    return _AlignedTable()


def _aligned_tables(n):
    """n tables in one buffer (one allocation for a batched call)."""
    buf = np.empty(n * _TABLE_SPAN, np.uint8)
    a0 = buf.ctypes.data
    return [_AlignedTable(buf, a0 + k * _TABLE_SPAN) for k in range(n)]


_lib = None


def lib():
    """Load libcheckers_amd.so once; raise if it is missing (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"checkers_amd: {LIB_PATH} not built; run `python -m checkers_amd.build`")
    L_ = ctypes.CDLL(LIB_PATH)
    u64, i32, vp = ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p
    sig = {
        "ckr_last_error": (ctypes.c_char_p, []),
        "ckr_version": (ctypes.c_char_p, []),
        "ckr_element_size": (i32, [i32]),
        "ckr_sidecar_bytes_per_elem": (i32, [i32]),
        "ckr_extract_mantissa": (i32, [vp, u64, i32, vp, vp, vp]),
        "ckr_byte_histogram": (i32, [vp, u64, i32, vp, vp]),
        "ckr_byte_histogram_raw": (i32, [vp, u64, vp, vp]),
        "ckr_byte_histogram_planes": (i32, [vp, u64, i32, vp, vp]),
        "ckr_build_table": (i32, [vp, i32, vp, vp]),
        "ckr_build_table_ranked": (i32, [vp, i32, vp, vp]),
        "ckr_build_tables_device": (i32, [vp, u64, i32, vp, vp]),
        "ckr_num_units": (u64, [u64, i32, u64]),
        "ckr_encode_max_output_bytes": (u64, [u64, i32, u64]),
        "ckr_encode_workspace_bytes": (u64, [u64, i32, u64]),
        "ckr_encode": (i32, [vp, u64, i32, vp, u64, vp, u64, vp, vp, vp, vp, u64, vp, vp]),
        "ckr_encode_planes": (i32, [vp, u64, i32, vp, vp, u64, vp, u64, vp, vp, vp, vp, u64, vp, vp]),
        "ckr_compress": (i32, [vp, u64, i32, u64, i32, vp, u64, vp, vp, vp, vp, u64, vp, vp, vp]),
        "ckr_compress_many": (i32, [vp, u64, u64, i32, vp]),
        "ckr_decode_workspace_bytes": (u64, [u64, i32, u64]),
        "ckr_decode": (i32, [vp, vp, vp, vp, u64, i32, u64, vp, vp, vp, u64, vp, vp]),
        "ckr_decode_many": (i32, [vp, u64, u64, i32, vp]),
        "ckr_decode_noalloc": (i32, [vp, vp, vp, vp, u64, i32, u64, vp, vp, vp, vp]),
        "ckr_analyze_workspace_bytes": (u64, [vp, u64]),
        "ckr_analyze": (i32, [vp, u64, vp, u64, vp]),
        "ckr_set_fast_paths": (i32, [i32]),
        "ckr_profile_begin": (i32, []),
        "ckr_profile_end": (i32, [ctypes.c_char_p, u64]),
        "ckr_repair_masked_bits": (i32, [i32, i32]),
        "ckr_repair_bucket_count": (u64, [u64]),
        "ckr_repair_workspace_bytes": (u64, [u64, i32, i32, ctypes.c_uint32]),
        "ckr_repair_build": (i32, [vp, u64, i32, i32, ctypes.c_uint32, vp, vp, vp, vp, vp, vp, u64, vp]),
        "ckr_repair_apply": (i32, [vp, u64, i32, i32, vp, ctypes.c_uint32, vp, vp, vp, u64, vp]),
        "ckr_fingerprint_weights": (i32, [vp, u64, vp]),
        "ckr_cluster": (i32, [vp, vp, u64, vp, vp]),
        "ckr_ckpt_write": (i32, [ctypes.c_char_p, i32, vp, u64, u64, i32, vp, vp]),
        "ckr_ckpt_set_slice_bytes": (i32, [u64]),
        "ckr_ckpt_slice_bytes": (u64, []),
        "ckr_ckpt_reserve": (i32, [vp, u64, u64]),
        "ckr_ckpt_pool_bytes": (u64, []),
        "ckr_ckpt_release": (None, []),
        "ckr_ckpt_open": (i32, [ctypes.c_char_p, i32, vp]),
        "ckr_ckpt_count": (u64, [vp]),
        "ckr_ckpt_info": (i32, [vp, u64, vp]),
        "ckr_ckpt_restore": (i32, [vp, u64, vp, vp]),
        "ckr_ckpt_close": (None, [vp]),
        "ckr_arena_create": (i32, [u64, vp]),
        "ckr_arena_alloc": (i32, [vp, u64, u64, vp]),
        "ckr_arena_used": (u64, [vp]),
        "ckr_arena_reset": (None, [vp]),
        "ckr_arena_destroy": (None, [vp]),
        "ckr_stats_slab_bytes": (u64, [ctypes.c_uint32, u64]),
        "ckr_carve_stats_slab": (i32, [vp, ctypes.c_uint32, u64, vp]),
        "ckr_analyze_device_records": (i32, [vp, u64, vp, u64, vp]),
        "ckr_analyze_device_records_workspace_bytes": (u64, [vp, u64]),
        "ckr_make_contiguous": (i32, [vp, i32, vp, vp, i32, vp, vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L_, name)
        f.restype = res
        f.argtypes = args
    _lib = L_
    return _lib


def _check(rc):
    if rc != CKR_OK:
        raise CkrError(rc, lib().ckr_last_error().decode())


def set_fast_paths(mode):
    """1: fast kernels (default); 0: general kernels; 2: fast kernels with minimal
    LDS lane slots (overflow route through the general kernels); 3: the same
    slots, the overflowing units coded again by the fast encoder with slots
    that hold any lane.  Returns the previous mode."""
    return int(lib().ckr_set_fast_paths(int(mode)))


def profile_begin():
    _check(lib().ckr_profile_begin())


def profile_end():
    """{kernel: (launches, total_ms)} of the launches since profile_begin()."""
    buf = ctypes.create_string_buffer(1 << 16)
    _check(lib().ckr_profile_end(buf, len(buf)))
    out = {}
    for line in buf.value.decode().splitlines():
        name, cnt, ms = line.split()
        out[name] = (int(cnt), float(ms))
    return out


def element_size(dtype):
    return lib().ckr_element_size(dtype)


def sidecar_bytes_per_elem(dtype):
    return lib().ckr_sidecar_bytes_per_elem(dtype)


def num_units(n_elems, dtype, unit_bytes):
    return lib().ckr_num_units(n_elems, dtype, unit_bytes)


def build_table(hist, ensure_full_alphabet=False):
    """Host table from a 256-bin histogram (ANSCompressor::normalize_histogram)."""
    h = np.ascontiguousarray(np.asarray(hist, dtype=np.uint32))
    assert h.shape == (256,)
    t = aligned_table()
    s = ctypes.c_uint32(0)
    _check(lib().ckr_build_table(h.ctypes.data, int(bool(ensure_full_alphabet)), t.ptr, ctypes.byref(s)))
    return t, s.value


def build_table_ranked(hist, ensure_full_alphabet=False):
    """The same table by ranks, without the sort (ckr_build_table_ranked):
    (table, ambiguous); ambiguous: only the reference's sort order decides."""
    h = np.ascontiguousarray(np.asarray(hist, dtype=np.uint32))
    assert h.shape == (256,)
    t = aligned_table()
    amb = ctypes.c_int(0)
    _check(lib().ckr_build_table_ranked(h.ctypes.data, int(bool(ensure_full_alphabet)), t.ptr, ctypes.byref(amb)))
    return t, bool(amb.value)


def build_tables_device(d_hists, ensure_full_alphabet=False, stream=None):
    """n tables by ranks on the device from a (n, 256) uint32 (int32) device
    tensor: a (n, 258) tensor of rows {norm_freq[256], sum, ambiguity flag}."""
    torch = _torch()
    assert d_hists.dim() == 2 and d_hists.shape[1] == 256 and d_hists.element_size() == 4 and d_hists.is_contiguous()
    rows = torch.empty((d_hists.shape[0], 258), dtype=torch.int32, device=d_hists.device)
    _check(lib().ckr_build_tables_device(d_hists.data_ptr(), d_hists.shape[0], int(bool(ensure_full_alphabet)),
                                         rows.data_ptr(), _stream(stream)))
    return rows


# --------------------------------------------------------------- torch helpers
def _torch():
    import torch
    return torch


def torch_tag(dtype):
    """C tag of a torch dtype (explicit; checkers_py parses dtype strings as the reference does)."""
    torch = _torch()
    return {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.int8: I8,
            torch.int32: I32}.get(dtype, UNKNOWN)


def _stream(stream):
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _n_elems(src, dtype, n_elems):
    """Element count of `src` read as `dtype` (from its byte size), or n_elems if given;
    never more elements than the tensor's bytes hold."""
    es = element_size(dtype)
    if es == 0:
        raise CkrError(CKR_E_INVALID, f"unknown dtype tag {dtype}")
    cap = src.numel() * src.element_size() // es
    if n_elems is None:
        return cap
    if n_elems > cap:
        raise CkrError(CKR_E_INVALID, f"n_elems={n_elems} exceeds the {cap} elements the tensor holds")
    return int(n_elems)


def _empty(nbytes, device):
    torch = _torch()
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


class Encoded:
    """Device-resident result of encode(): data[:total], headers, unit offsets, sidecar."""

    def __init__(self, data, headers, unit_offsets, sidecar, total, n_elems, dtype, unit_bytes, table):
        self.data, self.headers, self.unit_offsets, self.sidecar = data, headers, unit_offsets, sidecar
        self.total, self.n_elems, self.dtype, self.unit_bytes, self.table = total, n_elems, dtype, unit_bytes, table

    @property
    def n_units(self):
        return self.unit_offsets.numel() - 1

    def headers_np(self):
        return self.headers.cpu().numpy().view(HEADER_DTYPE).reshape(-1)

    def data_np(self):
        return self.data[: self.total].cpu().numpy()


class CompressJob(ctypes.Structure):
    _fields_ = [("d_src", ctypes.c_void_p), ("n_elems", ctypes.c_uint64), ("dtype", ctypes.c_int32),
                ("pad", ctypes.c_int32), ("d_out", ctypes.c_void_p), ("out_capacity", ctypes.c_uint64),
                ("d_headers", ctypes.c_void_p), ("d_unit_offsets", ctypes.c_void_p), ("d_sidecar", ctypes.c_void_p),
                ("d_workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_uint64), ("h_table", ctypes.c_void_p),
                ("total", ctypes.c_uint64)]


class Encoder:
    """Reusable buffers for repeated encodes of one tensor shape (bench / tests)."""

    def __init__(self, n_elems, dtype, unit_bytes, device="cuda"):
        torch = _torch()
        self.n_elems, self.dtype, self.unit_bytes = int(n_elems), dtype, int(unit_bytes)
        Lb = lib()
        es = Lb.ckr_element_size(dtype)
        if es == 0:
            raise CkrError(CKR_E_INVALID, f"unknown dtype tag {dtype}")
        self.n_bytes = self.n_elems * es
        self.n_units = int(Lb.ckr_num_units(self.n_elems, dtype, self.unit_bytes))
        self.ws_bytes = int(Lb.ckr_encode_workspace_bytes(self.n_elems, dtype, self.unit_bytes))
        self.out_cap = int(Lb.ckr_encode_max_output_bytes(self.n_elems, dtype, self.unit_bytes))
        self.ws = _empty(self.ws_bytes, device)
        self.out = _empty(self.out_cap, device)
        self.headers = torch.empty(max(self.n_units, 1) * LANES * 4, dtype=torch.int32, device=device)
        self.unit_offsets = torch.empty(self.n_units + 1, dtype=torch.int64, device=device)
        spe = Lb.ckr_sidecar_bytes_per_elem(dtype)
        self.sidecar = _empty(self.n_elems * spe, device) if spe else None
        self._make_job()

    # the buffers a compress_many job record points at: replacing one of them
    # rebuilds this encoder's record
    _JOB_BUFFERS = frozenset(("ws", "out", "out_cap", "headers", "unit_offsets", "sidecar", "ws_bytes"))

    def __setattr__(self, name, value):
        object.__setattr__(self, name, value)
        if name in Encoder._JOB_BUFFERS and "_job" in self.__dict__:
            self._make_job()

    def _make_job(self):
        """This encoder's part of a compress_many job record (all but the
        source and the table), copied into each call's records."""
        self._job = CompressJob(None, self.n_elems, self.dtype, 0, self.out.data_ptr(), self.out_cap,
                                self.headers.data_ptr(), self.unit_offsets.data_ptr(),
                                self.sidecar.data_ptr() if self.sidecar is not None else None,
                                self.ws.data_ptr(), self.ws_bytes, None, 0)
        self._job_addr = ctypes.addressof(self._job)

    def _check_src(self, src):
        if src.numel() * src.element_size() < self.n_bytes:
            raise CkrError(CKR_E_INVALID, f"source holds {src.numel() * src.element_size()} bytes, need {self.n_bytes}")

    def encode(self, src, table, stream=None, sync_total=True, planes=None):
        """ckr_encode under a given table; with planes (512 host uint32 words, the
        live-plane histograms of byte_histogram(..., planes=True)), ckr_encode_planes."""
        self._check_src(src)
        tot = ctypes.c_uint64(0)
        tail = (self.out.data_ptr(), self.out_cap, self.headers.data_ptr(), self.unit_offsets.data_ptr(),
                self.sidecar.data_ptr() if self.sidecar is not None else None,
                self.ws.data_ptr(), self.ws_bytes, ctypes.byref(tot) if sync_total else None, _stream(stream))
        if planes is None:
            _check(lib().ckr_encode(src.data_ptr(), self.n_elems, self.dtype, table.ptr, self.unit_bytes, *tail))
        else:
            pl = np.ascontiguousarray(planes, dtype=np.uint32)
            if pl.size != 512:
                raise CkrError(CKR_E_INVALID, "encode: planes must hold 512 words")
            _check(lib().ckr_encode_planes(src.data_ptr(), self.n_elems, self.dtype, table.ptr,
                                           pl.ctypes.data_as(ctypes.c_void_p), self.unit_bytes, *tail))
        return Encoded(self.out, self.headers, self.unit_offsets, self.sidecar,
                       tot.value if sync_total else None, self.n_elems, self.dtype, self.unit_bytes, table)

    def compress(self, src, ensure_full_alphabet=False, stream=None):
        self._check_src(src)
        tot = ctypes.c_uint64(0)
        t = aligned_table()
        _check(lib().ckr_compress(
            src.data_ptr(), self.n_elems, self.dtype, self.unit_bytes, int(bool(ensure_full_alphabet)),
            self.out.data_ptr(), self.out_cap, self.headers.data_ptr(), self.unit_offsets.data_ptr(),
            self.sidecar.data_ptr() if self.sidecar is not None else None,
            self.ws.data_ptr(), self.ws_bytes, t.ptr, ctypes.byref(tot), _stream(stream)))
        return Encoded(self.out, self.headers, self.unit_offsets, self.sidecar, tot.value, self.n_elems,
                       self.dtype, self.unit_bytes, t)


def compress_many(encoders, srcs, ensure_full_alphabet=False, stream=None):
    """ckr_compress_many: each (Encoder, source) pair compressed as Encoder.compress
    would, the next tensor's histogram overlapping the current one's encode.
    Every encoder must use the same unit size.  Returns one Encoded per pair."""
    if len(encoders) != len(srcs) or len({e.unit_bytes for e in encoders}) > 1:
        raise CkrError(CKR_E_INVALID, "compress_many: one source per encoder, all encoders of one unit size")
    if len({id(e) for e in encoders}) != len(encoders):
        raise CkrError(CKR_E_INVALID, "compress_many: an Encoder appears twice (its buffers would be shared)")
    if not encoders:
        return []
    n = len(encoders)
    jobs = (CompressJob * n)()
    tables = _aligned_tables(n)
    base, size = ctypes.addressof(jobs), ctypes.sizeof(CompressJob)
    for k, (e, src, t) in enumerate(zip(encoders, srcs, tables)):
        if src.nbytes < e.n_bytes:
            e._check_src(src)
        ctypes.memmove(base + k * size, e._job_addr, size)
        jb = jobs[k]
        jb.d_src, jb.h_table = src.data_ptr(), ctypes.addressof(t.table)
    _check(lib().ckr_compress_many(base, n, encoders[0].unit_bytes, int(bool(ensure_full_alphabet)),
                                   _stream(stream)))
    return [Encoded(e.out, e.headers, e.unit_offsets, e.sidecar, jb.total, e.n_elems, e.dtype, e.unit_bytes, t)
            for jb, e, t in zip(jobs, encoders, tables)]


def byte_histogram(src, dtype, n_elems=None, stream=None, planes=False):
    """256-bin histogram of the masked byte stream of `src` (torch device tensor);
    with planes=True, 768 bins: that histogram, then the two live planes'
    (ckr_byte_histogram_planes)."""
    torch = _torch()
    n = _n_elems(src, dtype, n_elems)
    h = torch.empty(768 if planes else 256, dtype=torch.int32, device=src.device)
    f = lib().ckr_byte_histogram_planes if planes else lib().ckr_byte_histogram
    _check(f(src.data_ptr(), n, dtype, h.data_ptr(), _stream(stream)))
    return h


def extract_mantissa(src, dtype, n_elems=None, stream=None):
    torch = _torch()
    n = _n_elems(src, dtype, n_elems)
    es, spe = element_size(dtype), sidecar_bytes_per_elem(dtype)
    masked = torch.empty(max(n * es, 1), dtype=torch.uint8, device=src.device)
    side = torch.empty(max(n * spe, 1), dtype=torch.uint8, device=src.device)
    _check(lib().ckr_extract_mantissa(src.data_ptr(), n, dtype, masked.data_ptr(), side.data_ptr(), _stream(stream)))
    return masked[: n * es], side[: n * spe]


def encode(src, dtype, table, unit_bytes, n_elems=None, stream=None):
    n = _n_elems(src, dtype, n_elems)
    enc = Encoder(n, dtype, unit_bytes, device=src.device)
    return enc.encode(src, table, stream=stream)


def compress(src, dtype, unit_bytes, ensure_full_alphabet=False, n_elems=None, stream=None):
    n = _n_elems(src, dtype, n_elems)
    return Encoder(n, dtype, unit_bytes, device=src.device).compress(src, ensure_full_alphabet, stream=stream)


class Decoder:
    def __init__(self, n_elems, dtype, unit_bytes, device="cuda"):
        self.n_elems, self.dtype, self.unit_bytes = int(n_elems), dtype, int(unit_bytes)
        self.ws_bytes = int(lib().ckr_decode_workspace_bytes(self.n_elems, dtype, self.unit_bytes))
        self.ws = _empty(self.ws_bytes, device)

    def decode(self, data, headers, unit_offsets, table, sidecar, dst, stream=None, check=True):
        bad = ctypes.c_uint64(0)
        _check(lib().ckr_decode(
            data.data_ptr(), headers.data_ptr(), unit_offsets.data_ptr(), table.ptr, self.n_elems, self.dtype,
            self.unit_bytes, sidecar.data_ptr() if sidecar is not None else None, dst.data_ptr(),
            self.ws.data_ptr(), self.ws_bytes, ctypes.byref(bad) if check else None, _stream(stream)))
        return bad.value if check else None


class DecodeJob(ctypes.Structure):
    _fields_ = [("d_data", ctypes.c_void_p), ("d_headers", ctypes.c_void_p), ("d_unit_offsets", ctypes.c_void_p),
                ("h_table", ctypes.c_void_p), ("n_elems", ctypes.c_uint64), ("dtype", ctypes.c_int32),
                ("pad", ctypes.c_int32), ("d_sidecar", ctypes.c_void_p), ("d_dst", ctypes.c_void_p),
                ("d_workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_uint64), ("bad_lanes", ctypes.c_uint64)]


def decode_many(decoders, encoded, dsts, check=True, stream=None):
    """ckr_decode_many: encoded[k] (an Encoded, or any object with data,
    headers, unit_offsets, table and sidecar) decoded by decoders[k] into
    dsts[k], as Decoder.decode would; a shard of small tensors is decoded by one
    set-up and one decode launch per dtype class (side by side on several
    streams when the fast decoder does not take every job whole).  Returns the
    bad-lane counts (None when check is False)."""
    if not (len(decoders) == len(encoded) == len(dsts)) or len({d.unit_bytes for d in decoders}) > 1:
        raise CkrError(CKR_E_INVALID, "decode_many: one item and destination per decoder, one unit size")
    if len({id(d) for d in decoders}) != len(decoders):
        raise CkrError(CKR_E_INVALID, "decode_many: a Decoder appears twice (its workspace would be shared)")
    if not decoders:
        return [] if check else None
    jobs = (DecodeJob * len(decoders))()
    for jb, d, e, dst in zip(jobs, decoders, encoded, dsts):
        jb.d_data, jb.d_headers, jb.d_unit_offsets = e.data.data_ptr(), e.headers.data_ptr(), e.unit_offsets.data_ptr()
        jb.h_table, jb.n_elems, jb.dtype = ctypes.addressof(e.table.table), d.n_elems, d.dtype
        jb.d_sidecar = e.sidecar.data_ptr() if e.sidecar is not None else None
        jb.d_dst, jb.d_workspace, jb.workspace_bytes = dst.data_ptr(), d.ws.data_ptr(), d.ws_bytes
    _check(lib().ckr_decode_many(ctypes.addressof(jobs), len(decoders), decoders[0].unit_bytes, int(bool(check)),
                                 _stream(stream)))
    return [jb.bad_lanes for jb in jobs] if check else None


def decode(enc, dst=None, stream=None):
    """Decode an Encoded back into original bytes; returns (dst uint8 tensor, bad_lanes)."""
    torch = _torch()
    nb = enc.n_elems * element_size(enc.dtype)
    if dst is None:
        dst = torch.empty(max(nb, 1), dtype=torch.uint8, device=enc.data.device)
    d = Decoder(enc.n_elems, enc.dtype, enc.unit_bytes, device=enc.data.device)
    bad = d.decode(enc.data, enc.headers, enc.unit_offsets, enc.table, enc.sidecar, dst, stream=stream)
    return dst[:nb], bad


def decode_noalloc(enc, dst, stream=None, check=True):
    """ckr_decode_noalloc: decode an Encoded into dst (a 4-byte aligned device
    tensor of its byte size) with no device allocation; returns the bad-lane
    count (None when check is False)."""
    bad = ctypes.c_uint64(0)
    _check(lib().ckr_decode_noalloc(
        enc.data.data_ptr(), enc.headers.data_ptr(), enc.unit_offsets.data_ptr(), enc.table.ptr, enc.n_elems,
        enc.dtype, enc.unit_bytes, enc.sidecar.data_ptr() if enc.sidecar is not None else None, dst.data_ptr(),
        ctypes.byref(bad) if check else None, _stream(stream)))
    return bad.value if check else None


class Analyzer:
    """ckr_analyze over a fixed list of device tensors, with its outputs and
    workspace allocated once: run() enqueues the statistics pass on the stream
    (no synchronisation), results() waits and copies them to the host."""

    def __init__(self, tensors, tags, bins=256):
        torch = _torch()
        n = len(tensors)
        dev = tensors[0].device if n else "cuda"
        self.n, self.nb = n, min(bins, 256)
        self.hist = torch.zeros((max(n, 1), max(self.nb, 1)), dtype=torch.int32, device=dev)
        self.mom = torch.zeros((max(n, 1), 4), dtype=torch.float32, device=dev)
        self.mm = torch.zeros((max(n, 1), 2), dtype=torch.float32, device=dev)
        self.fp = torch.zeros((max(n, 1), 5), dtype=torch.float32, device=dev)
        self.tensors = list(tensors)
        self.recs = (StatsRecord * max(n, 1))()
        for i, (t, tag) in enumerate(zip(tensors, tags)):
            ne = _n_elems(t, tag, None)
            self.recs[i].d_ptr = t.data_ptr() if ne else None
            self.recs[i].num_elements = ne
            self.recs[i].histogram_bins = bins
            self.recs[i].data_type = tag
            self.recs[i].d_histogram = self.hist[i].data_ptr()
            self.recs[i].d_raw_moments = self.mom[i].data_ptr()
            self.recs[i].d_minmax = self.mm[i].data_ptr()
            self.recs[i].d_fingerprint = self.fp[i].data_ptr()
        self.wsb = int(lib().ckr_analyze_workspace_bytes(self.recs, n))
        self.ws = _empty(self.wsb, dev)

    def run(self, stream=None):
        _check(lib().ckr_analyze(self.recs, self.n, self.ws.data_ptr(), self.wsb, _stream(stream)))

    def results(self):
        _torch().cuda.synchronize()
        return [dict(histogram=self.hist[i, :self.nb].cpu().numpy().view(np.uint32).copy(),
                     moments=self.mom[i].cpu().numpy().copy(), minmax=self.mm[i].cpu().numpy().copy(),
                     fingerprint=self.fp[i].cpu().numpy().copy()) for i in range(self.n)]


def analyze(tensors, tags, bins=256, stream=None):
    """TensorAnalyzer statistics for a list of device tensors.

    Returns a list of dicts with histogram (np.uint32), moments (mean, var,
    skew, kurt), minmax and fingerprint, all copied to the host."""
    a = Analyzer(tensors, tags, bins)
    a.run(stream)
    return a.results()


# ---- tensor-group prefix-mask repair
class RepairRule(ctypes.Structure):
    """SharedGrammarRule (tensor_group_prefix_mask_repair.cpp:70-75)."""
    _fields_ = [("replacement", ctypes.c_uint64), ("lhs", ctypes.c_uint64), ("rhs", ctypes.c_uint64),
                ("frequency", ctypes.c_uint64)]


def repair_masked_bits(dtype, request=None):
    """Masked mantissa bits used for a dtype (request None: all mantissa bits)."""
    k = int(lib().ckr_repair_masked_bits(dtype, -1 if request is None else int(request)))
    if k < 0:
        raise CkrError(CKR_E_INVALID, f"Unsupported dtype for mantissa-mask compression: tag {dtype}")
    return k


def repair_bucket_count(n):
    return int(lib().ckr_repair_bucket_count(n))


class Repairer:
    """Workspace holder for build_shared_grammar / apply_existing_grammar on
    device tensors of at most n_elems words."""

    def __init__(self, n_elems, dtype, masked_bits=None, max_rules=50, device="cuda"):
        self.n, self.dtype, self.max_rules = int(n_elems), dtype, int(max_rules)
        self.mb = -1 if masked_bits is None else int(masked_bits)
        repair_masked_bits(dtype, masked_bits)
        wsb = int(lib().ckr_repair_workspace_bytes(self.n, dtype, self.mb, self.max_rules))
        if wsb == 0:
            raise CkrError(CKR_E_INVALID, lib().ckr_last_error().decode())
        self.wsb = wsb
        self.ws = _empty(wsb, device)

    def build(self, src, want_seq=False, stream=None):
        """dict(rules=[(replacement, lhs, rhs, freq)], out_len, max_pair[, seq])."""
        torch = _torch()
        n = _n_elems(src, self.dtype, None)
        if n > self.n:
            raise CkrError(CKR_E_INVALID, f"tensor of {n} words exceeds the workspace's {self.n}")
        rules = (RepairRule * max(self.max_rules, 1))()
        nr, out_len, mp = ctypes.c_uint32(0), ctypes.c_uint64(0), ctypes.c_uint64(0)
        seq = torch.empty(max(n, 1), dtype=torch.int64, device=src.device) if want_seq else None
        _check(lib().ckr_repair_build(src.data_ptr() if n else None, n, self.dtype, self.mb, self.max_rules,
                                      rules, ctypes.byref(nr), ctypes.byref(out_len), ctypes.byref(mp),
                                      seq.data_ptr() if want_seq else None, self.ws.data_ptr(), self.wsb,
                                      _stream(stream)))
        r = dict(rules=[(rules[i].replacement, rules[i].lhs, rules[i].rhs, rules[i].frequency)
                        for i in range(nr.value)], out_len=out_len.value, max_pair=mp.value)
        if want_seq:
            r["seq"] = seq[: out_len.value].cpu().numpy().view(np.uint64)
        return r

    def apply(self, src, rules, want_seq=False, stream=None):
        """Token count after applying the rules in order (and the sequence)."""
        torch = _torch()
        n = _n_elems(src, self.dtype, None)
        if n > self.n or len(rules) > self.max_rules:
            raise CkrError(CKR_E_INVALID, "tensor or rule list exceeds the workspace")
        rr = (RepairRule * max(len(rules), 1))()
        for i, (rep, lhs, rhs, f) in enumerate(rules):
            rr[i].replacement, rr[i].lhs, rr[i].rhs, rr[i].frequency = rep, lhs, rhs, f
        out_len = ctypes.c_uint64(0)
        seq = torch.empty(max(n, 1), dtype=torch.int64, device=src.device) if want_seq else None
        _check(lib().ckr_repair_apply(src.data_ptr() if n else None, n, self.dtype, self.mb, rr, len(rules),
                                      ctypes.byref(out_len), seq.data_ptr() if want_seq else None,
                                      self.ws.data_ptr(), self.wsb, _stream(stream)))
        if want_seq:
            return out_len.value, seq[: out_len.value].cpu().numpy().view(np.uint64)
        return out_len.value


# ---- fingerprint weights, clusters, rank checkpoint files
def fingerprint_weights(fingerprints):
    """compute_fingerprint_weights: 5 weights from n x 5 fingerprints."""
    fp = np.ascontiguousarray(np.asarray(fingerprints, np.float32).reshape(-1, 5))
    w = np.zeros(5, np.float64)
    _check(lib().ckr_fingerprint_weights(fp.ctypes.data, fp.shape[0], w.ctypes.data))
    return w


def cluster(names, fingerprints):
    """build_knn_clusters: (cluster id per record, -1 for singletons; thresholds
    of the non-empty categories in name order)."""
    fp = np.ascontiguousarray(np.asarray(fingerprints, np.float32).reshape(-1, 5))
    n = fp.shape[0]
    arr = (ctypes.c_char_p * max(n, 1))(*[x.encode() for x in names])
    out = np.zeros(max(n, 1), np.int32)
    thr = np.zeros(4, np.float64)
    _check(lib().ckr_cluster(arr, fp.ctypes.data, n, out.ctypes.data, thr.ctypes.data))
    ncat = len({_category(x) for x in names})
    return out[:n].tolist(), thr[:ncat].tolist()


def _category(name):
    for p, c in (("optimizer.exp_avg_sq::", "exp_avg_sq"), ("optimizer.exp_avg::", "exp_avg"),
                 ("master_weights::", "master_weights")):
        if name.startswith(p):
            return c
    return "model_state"


class CkptTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("d_ptr", ctypes.c_void_p), ("num_elements", ctypes.c_uint64),
                ("dtype", ctypes.c_int32), ("cluster_id", ctypes.c_int32)]


class CkptStats(ctypes.Structure):
    _fields_ = [("record_index", ctypes.c_uint64), ("original_bytes", ctypes.c_uint64),
                ("ans_bytes", ctypes.c_uint64), ("sidecar_bytes", ctypes.c_uint64),
                ("owns_table", ctypes.c_uint32), ("table_sum", ctypes.c_uint32),
                ("table_repaired", ctypes.c_uint32), ("n_slices", ctypes.c_uint32),
                ("stored_bytes", ctypes.c_uint64), ("record_bytes", ctypes.c_uint64),
                ("hist_ms", ctypes.c_double), ("table_ms", ctypes.c_double),
                ("encode_ms", ctypes.c_double), ("copy_ms", ctypes.c_double)]


class CkptEntry(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("anchor_name", ctypes.c_char * 256),
                ("dtype", ctypes.c_uint32), ("is_raw", ctypes.c_uint32), ("owns_table", ctypes.c_uint32),
                ("version", ctypes.c_uint32), ("original_bytes", ctypes.c_uint64),
                ("num_elements", ctypes.c_uint64), ("data_size", ctypes.c_uint64), ("n_units", ctypes.c_uint64),
                ("unit_bytes", ctypes.c_uint64), ("sidecar_bytes", ctypes.c_uint64)]


def _ckpt_tensors(tensors):
    n = len(tensors)
    names = [t[0].encode() for t in tensors]
    arr = (CkptTensor * max(n, 1))()
    for i, (name, t, tag, cid) in enumerate(tensors):
        ne = _n_elems(t, tag, None) if t is not None else 0
        arr[i].name = names[i]
        arr[i].d_ptr = t.data_ptr() if (t is not None and ne) else None
        arr[i].num_elements = ne
        arr[i].dtype = tag
        arr[i].cluster_id = cid
    return arr, names


def set_ckpt_slice_bytes(nbytes):
    """Slice size of the checkpoint writer (0: CKR_CKPT_SLICE_BYTES or 4 GiB)."""
    _check(lib().ckr_ckpt_set_slice_bytes(nbytes))


def ckpt_slice_bytes():
    return int(lib().ckr_ckpt_slice_bytes())


def reserve_checkpoint(tensors, unit_bytes=0):
    """Allocate the writer's buffers for these tensors ahead of write_checkpoint."""
    arr, _names = _ckpt_tensors(tensors)
    _check(lib().ckr_ckpt_reserve(arr, len(tensors), unit_bytes))


def ckpt_pool_bytes():
    return int(lib().ckr_ckpt_pool_bytes())


def release_checkpoint_buffers():
    lib().ckr_ckpt_release()


def write_checkpoint(output_dir, rank, tensors, unit_bytes=0, repair_tables=False, stream=None):
    """compress_and_save_all: tensors is a list of (name, device tensor or None,
    dtype tag, cluster id); returns one stats dict per written tensor."""
    n = len(tensors)
    arr, _names = _ckpt_tensors(tensors)
    st = (CkptStats * max(n, 1))()
    _check(lib().ckr_ckpt_write(os.fsencode(output_dir), rank, arr, n, unit_bytes, int(bool(repair_tables)), st,
                                _stream(stream)))
    written = sum(1 for i in range(n) if arr[i].d_ptr and arr[i].num_elements)
    return [{f[0]: getattr(st[i], f[0]) for f in CkptStats._fields_} for i in range(written)]


class Checkpoint:
    """Reader of a rank's .ansc (v2 or v4) / .mant / .dict files; restores
    tensors on the device."""

    def __init__(self, directory, rank=0):
        self._h = ctypes.c_void_p()
        _check(lib().ckr_ckpt_open(os.fsencode(directory), rank, ctypes.byref(self._h)))

    def __len__(self):
        return int(lib().ckr_ckpt_count(self._h))

    def info(self, i):
        e = CkptEntry()
        _check(lib().ckr_ckpt_info(self._h, i, ctypes.byref(e)))
        d = {f[0]: getattr(e, f[0]) for f in CkptEntry._fields_}
        d["name"] = e.name.decode()
        d["anchor_name"] = e.anchor_name.decode()
        return d

    def restore(self, i, dst=None, device="cuda", stream=None):
        """Decode tensor i into dst (a device tensor of its byte size; a new
        uint8 tensor when None); returns dst."""
        torch = _torch()
        info = self.info(i)
        if dst is None:
            dst = torch.empty(max(info["original_bytes"], 1), dtype=torch.uint8, device=device)
        elif dst.numel() * dst.element_size() < info["original_bytes"]:
            raise CkrError(CKR_E_CAPACITY, "destination too small")
        _check(lib().ckr_ckpt_restore(self._h, i, dst.data_ptr(), _stream(stream)))
        return dst

    def close(self):
        if self._h:
            lib().ckr_ckpt_close(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
