"""The context layer of the C ABI (ckr_context.hip): the 72-byte device record,
the arena, the statistics slab carving (src/MemoryManager.cpp:403-481,
:692-707) and the strided gather of TensorResource::make_contiguous
(src/TensorResource.cpp:85-153)."""
import ctypes

import pytest

import checkers_amd as ck


class DeviceTensorRecord(ctypes.Structure):
    # include/checkers/MemoryManager.hpp:60-72
    _fields_ = [("name", ctypes.c_char_p), ("d_ptr", ctypes.c_void_p), ("d_histogram", ctypes.c_void_p),
                ("d_raw_moments", ctypes.c_void_p), ("d_statistics", ctypes.c_void_p),
                ("d_fingerprint", ctypes.c_void_p), ("d_minmax", ctypes.c_void_p),
                ("num_elements", ctypes.c_uint64), ("histogram_bins", ctypes.c_uint32),
                ("data_type", ctypes.c_uint8), ("contiguity", ctypes.c_uint8), ("pad_", ctypes.c_uint8 * 2)]


def test_record_layout_and_slab_plan():
    assert ctypes.sizeof(DeviceTensorRecord) == 72
    assert DeviceTensorRecord.num_elements.offset == 56 and DeviceTensorRecord.data_type.offset == 68
    L = ck.lib()
    # compute_buffer_plan: bins*4, 16 B moments, 8 B min/max, 20 B fingerprint, each aligned
    assert L.ckr_stats_slab_bytes(256, 256) == 1024 + 256 + 256 + 256
    assert L.ckr_stats_slab_bytes(300, 256) == 1280 + 3 * 256
    assert L.ckr_stats_slab_bytes(256, 1) == 1024 + 16 + 8 + 20
    r = DeviceTensorRecord()
    base = 0x7F0000000000   # carving only computes addresses
    assert L.ckr_carve_stats_slab(ctypes.c_void_p(base), 300, 256, ctypes.byref(r)) == ck.CKR_OK
    assert (r.d_histogram, r.d_raw_moments, r.d_minmax, r.d_fingerprint) == (
        base, base + 1280, base + 1536, base + 1792)
    assert r.d_statistics is None and r.histogram_bins == 300
    assert L.ckr_carve_stats_slab(ctypes.c_void_p(base), 256, 24, ctypes.byref(r)) == ck.CKR_E_INVALID


def test_gather_argument_errors():
    L = ck.lib()
    shape = (ctypes.c_int64 * 9)(*([2] * 9))
    strides = (ctypes.c_int64 * 9)(*([1] * 9))
    assert L.ckr_make_contiguous(None, 9, shape, strides, 4, None, None) == ck.CKR_E_INVALID
    assert L.ckr_make_contiguous(None, 2, shape, strides, 3, None, None) == ck.CKR_E_INVALID
    neg = (ctypes.c_int64 * 2)(4, -1)
    assert L.ckr_make_contiguous(None, 2, shape, neg, 4, None, None) == ck.CKR_E_INVALID
    zero = (ctypes.c_int64 * 2)(0, 5)
    assert L.ckr_make_contiguous(None, 2, zero, strides, 4, None, None) == ck.CKR_OK   # nothing to copy


@pytest.mark.gpu
def test_arena_bump_allocation(gpu):
    L = ck.lib()
    a = ctypes.c_void_p()
    assert L.ckr_arena_create(1 << 20, ctypes.byref(a)) == ck.CKR_OK, L.ckr_last_error()
    try:
        p1, p2, p3 = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        assert L.ckr_arena_alloc(a, 100, 256, ctypes.byref(p1)) == ck.CKR_OK
        assert L.ckr_arena_alloc(a, 10, 512, ctypes.byref(p2)) == ck.CKR_OK
        assert p1.value % 256 == 0 and p2.value % 512 == 0 and p2.value - p1.value == 512
        assert L.ckr_arena_used(a) == 522
        assert L.ckr_arena_alloc(a, 8, 3, ctypes.byref(p3)) == ck.CKR_E_INVALID
        assert L.ckr_arena_alloc(a, 1 << 20, 256, ctypes.byref(p3)) == ck.CKR_E_CAPACITY
        L.ckr_arena_reset(a)
        assert L.ckr_arena_alloc(a, 1 << 20, 256, ctypes.byref(p3)) == ck.CKR_OK and p3.value == p1.value
    finally:
        L.ckr_arena_destroy(a)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,make", [
    ("float32", lambda t: t.t()),                                # transposed 2-D
    ("bfloat16", lambda t: t[:, ::3]),                            # column step
    ("int8", lambda t: t.reshape(6, 10, 12).permute(2, 0, 1)),    # 3-D permutation
    ("float64", lambda t: t[1:, 2:7]),                            # offset window
    ("float32", lambda t: t.reshape(60, 12)[:, :1].expand(60, 5)),  # zero stride
])
def test_make_contiguous_matches_torch(gpu, dtype, make):
    import torch
    dt = getattr(torch, dtype)
    base = (torch.arange(720, device=gpu) % 251).to(dt).reshape(60, 12)
    v = make(base)
    out = torch.full((v.numel(),), 7, dtype=dt, device=gpu)
    shape = (ctypes.c_int64 * v.dim())(*v.shape)
    strides = (ctypes.c_int64 * v.dim())(*v.stride())
    rc = ck.lib().ckr_make_contiguous(ctypes.c_void_p(v.data_ptr()), v.dim(), shape, strides, v.element_size(),
                                      ctypes.c_void_p(out.data_ptr()), torch.cuda.current_stream().cuda_stream)
    assert rc == ck.CKR_OK, ck.lib().ckr_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, v.contiguous().reshape(-1))


@pytest.mark.gpu
def test_make_contiguous_rejects_out_of_range_source(gpu):
    """A stride vector that reaches past the source's allocation is refused
    before launch (hipMemGetAddressRange bounds it); host memory likewise."""
    import numpy as np
    import torch
    hip = ctypes.CDLL("libamdhip64.so")
    d = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(d), ctypes.c_size_t(1 << 20)) == 0
    out = torch.zeros(100, dtype=torch.float32, device=gpu)
    try:
        src = ctypes.c_void_p(d.value + (1 << 20) - 400)   # the last 100 floats of the allocation
        shape = (ctypes.c_int64 * 2)(10, 10)
        inside = (ctypes.c_int64 * 2)(10, 1)
        past = (ctypes.c_int64 * 2)(20, 1)        # last element 189 of a 100-element allocation
        L = ck.lib()
        assert L.ckr_make_contiguous(src, 2, shape, past, 4, ctypes.c_void_p(out.data_ptr()), None) == ck.CKR_E_INVALID
        assert b"past its allocation" in L.ckr_last_error()
        host = np.zeros(100, np.float32)
        assert L.ckr_make_contiguous(ctypes.c_void_p(host.ctypes.data), 2, shape, inside, 4,
                                     ctypes.c_void_p(out.data_ptr()), None) == ck.CKR_E_INVALID
        assert L.ckr_make_contiguous(src, 2, shape, inside, 4, ctypes.c_void_p(out.data_ptr()), None) == ck.CKR_OK
        torch.cuda.synchronize()
    finally:
        hip.hipFree(d)
