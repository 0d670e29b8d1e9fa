// checkers_amd/csrc/ckr_context.hip — the memory side of the context layer:
// the per-tensor device record, a hipMalloc arena for the statistics slabs and
// for contiguous copies, the slab carving, and the strided gather.
//
// Reference (paths relative to the reference tree):
//   DeviceTensorRecord                      include/checkers/MemoryManager.hpp:60-72
//   BufferPlan / compute_buffer_plan        include/checkers/MemoryManager.hpp:77-84, src/MemoryManager.cpp:692-707
//   slab carving (STEP 3/4 of a batch)      src/MemoryManager.cpp:403-481
//   TensorResource::make_contiguous         src/TensorResource.cpp:85-153
// The reference allocates its slabs and copies from Umpire pools and runs the
// gather as a RAJA forall; here one hipMalloc'd arena serves every slab and
// copy of a context, and the gather is a HIP kernel over the full stride vector.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstddef>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "checkers_amd.h"
#include "ckr_internal.h"

static_assert(sizeof(ckr_device_tensor_record) == 72, "DeviceTensorRecord is 72 bytes");
static_assert(offsetof(ckr_device_tensor_record, num_elements) == 56, "DeviceTensorRecord layout");
static_assert(offsetof(ckr_device_tensor_record, histogram_bins) == 64, "DeviceTensorRecord layout");
static_assert(offsetof(ckr_device_tensor_record, data_type) == 68, "DeviceTensorRecord layout");
static_assert(offsetof(ckr_device_tensor_record, contiguity) == 69, "DeviceTensorRecord layout");

struct ckr_arena {
    uint8_t* base = nullptr;
    uint64_t capacity = 0;
    uint64_t used = 0;
};

namespace {

int err(int code, const std::string& m) { return ckr::set_error(code, m); }

inline uint64_t align_up(uint64_t v, uint64_t a) { return a ? (v + a - 1) / a * a : v; }

constexpr int kMaxDims = 8;
struct GatherArgs {
    int ndim;
    int es;
    uint64_t n;
    uint64_t shape[kMaxDims];
    int64_t stride[kMaxDims];  // elements
};

// One thread per element of the contiguous (row-major) output: its source
// element is the sum over dimensions of index x stride.
template <typename T>
__global__ void __launch_bounds__(256) gather_kernel(const T* __restrict__ src, T* __restrict__ dst, GatherArgs a) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t rem = i;
        int64_t off = 0;
        for (int d = a.ndim - 1; d >= 0; d--) {
            const uint64_t idx = rem % a.shape[d];
            rem /= a.shape[d];
            off += (int64_t)idx * a.stride[d];
        }
        dst[i] = src[off];
    }
}

std::vector<ckr_stats_record> stats_records(const ckr_device_tensor_record* h_recs, uint64_t n) {
    std::vector<ckr_stats_record> r(n);
    for (uint64_t i = 0; i < n; i++) {
        r[i].d_ptr = h_recs[i].d_ptr;
        r[i].num_elements = h_recs[i].num_elements;
        r[i].histogram_bins = h_recs[i].histogram_bins;
        r[i].data_type = h_recs[i].data_type;
        r[i].d_histogram = h_recs[i].d_histogram;
        r[i].d_raw_moments = h_recs[i].d_raw_moments;
        r[i].d_minmax = h_recs[i].d_minmax;
        r[i].d_fingerprint = h_recs[i].d_fingerprint;
    }
    return r;
}

}  // namespace

extern "C" {

int ckr_arena_create(uint64_t capacity, ckr_arena** out) {
    if (!out) return err(CKR_E_INVALID, "[ckr] null arena output");
    *out = nullptr;
    auto* a = new (std::nothrow) ckr_arena();
    if (!a) return err(CKR_E_CAPACITY, "[ckr] arena descriptor allocation failed");
    if (capacity) {
        const hipError_t e = hipMalloc(reinterpret_cast<void**>(&a->base), capacity);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            delete a;
            return err(CKR_E_HIP, std::string("[ckr] arena hipMalloc failed: ") + hipGetErrorString(e));
        }
    }
    a->capacity = capacity;
    *out = a;
    return CKR_OK;
}

int ckr_arena_alloc(ckr_arena* a, uint64_t bytes, uint64_t alignment, void** d_out) {
    if (!a || !d_out) return err(CKR_E_INVALID, "[ckr] null arena or output");
    if (alignment == 0 || (alignment & (alignment - 1))) return err(CKR_E_INVALID, "[ckr] alignment must be a power of two");
    const uint64_t off = align_up(a->used, alignment);
    if (off > a->capacity || bytes > a->capacity - off)
        return err(CKR_E_CAPACITY, "[ckr] arena full: " + std::to_string(bytes) + " bytes requested, " +
                                       std::to_string(a->capacity - std::min(off, a->capacity)) + " left");
    *d_out = a->base + off;
    a->used = off + bytes;
    return CKR_OK;
}

uint64_t ckr_arena_used(const ckr_arena* a) { return a ? a->used : 0; }

void ckr_arena_reset(ckr_arena* a) {
    if (a) a->used = 0;
}

void ckr_arena_destroy(ckr_arena* a) {
    if (!a) return;
    if (a->base) (void)hipFree(a->base);
    delete a;
}

uint64_t ckr_stats_slab_bytes(uint32_t histogram_bins, uint64_t alignment) {
    // compute_buffer_plan: the histogram slab holds all requested bins (the
    // kernel writes at most 256 of them), then 4 moments, min/max and the 5-float
    // fingerprint, each rounded up to the alignment
    return align_up((uint64_t)histogram_bins * 4, alignment) + align_up(16, alignment) + align_up(8, alignment) +
           align_up(20, alignment);
}

int ckr_carve_stats_slab(void* d_slab, uint32_t histogram_bins, uint64_t alignment, ckr_device_tensor_record* rec) {
    if (!d_slab || !rec) return err(CKR_E_INVALID, "[ckr] null slab or record");
    if (alignment && (alignment & (alignment - 1))) return err(CKR_E_INVALID, "[ckr] alignment must be a power of two");
    uint8_t* p = static_cast<uint8_t*>(d_slab);
    uint64_t cursor = 0;
    rec->d_histogram = reinterpret_cast<uint32_t*>(p + cursor);
    cursor += align_up((uint64_t)histogram_bins * 4, alignment);
    rec->d_raw_moments = reinterpret_cast<float*>(p + cursor);
    cursor += align_up(16, alignment);
    rec->d_minmax = reinterpret_cast<float*>(p + cursor);
    cursor += align_up(8, alignment);
    rec->d_fingerprint = reinterpret_cast<float*>(p + cursor);
    rec->d_statistics = nullptr;  // never set by the reference either (MemoryManager.cpp:468-480)
    rec->histogram_bins = histogram_bins;
    return CKR_OK;
}

int ckr_analyze_device_records(const ckr_device_tensor_record* h_recs, uint64_t n, void* d_workspace,
                               uint64_t workspace_bytes, void* stream) {
    if (n && !h_recs) return err(CKR_E_INVALID, "[ckr] null records");
    const std::vector<ckr_stats_record> r = stats_records(h_recs, n);
    return ckr_analyze(r.data(), n, d_workspace, workspace_bytes, stream);
}

uint64_t ckr_analyze_device_records_workspace_bytes(const ckr_device_tensor_record* h_recs, uint64_t n) {
    if (n && !h_recs) return 0;
    const std::vector<ckr_stats_record> r = stats_records(h_recs, n);
    return ckr_analyze_workspace_bytes(r.data(), n);
}

int ckr_make_contiguous(const void* d_src, int ndim, const int64_t* shape, const int64_t* strides, int elem_size,
                        void* d_dst, void* stream) {
    if (ndim < 0 || ndim > kMaxDims) return err(CKR_E_INVALID, "[ckr] make_contiguous supports up to 8 dimensions");
    if (elem_size != 1 && elem_size != 2 && elem_size != 4 && elem_size != 8)
        return err(CKR_E_INVALID, "[ckr] element size must be 1, 2, 4 or 8 bytes");
    if (ndim && (!shape || !strides)) return err(CKR_E_INVALID, "[ckr] null shape or strides");
    GatherArgs a{};
    a.ndim = ndim;
    a.es = elem_size;
    a.n = 1;
    int64_t max_off = 0;
    for (int d = 0; d < ndim; d++) {
        if (shape[d] < 0 || strides[d] < 0) return err(CKR_E_INVALID, "[ckr] negative shape or stride");
        a.shape[d] = (uint64_t)shape[d];
        a.stride[d] = strides[d];
        a.n *= (uint64_t)shape[d];
        if (shape[d] > 0) max_off += (shape[d] - 1) * strides[d];
    }
    if (a.n == 0) return CKR_OK;
    if (!d_src || !d_dst) return err(CKR_E_INVALID, "[ckr] null source or destination");
    if ((reinterpret_cast<uintptr_t>(d_src) | reinterpret_cast<uintptr_t>(d_dst)) % (uintptr_t)elem_size)
        return err(CKR_E_INVALID, "[ckr] source and destination must be aligned to the element size");
    // both ranges inside their allocations before anything is launched
    for (int which = 0; which < 2; which++) {
        const void* p = which ? d_dst : d_src;
        const uint64_t bytes = which ? a.n * (uint64_t)elem_size : ((uint64_t)max_off + 1) * (uint64_t)elem_size;
        hipPointerAttribute_t at;
        std::memset(&at, 0, sizeof(at));
        if (hipPointerGetAttributes(&at, p) != hipSuccess || at.type == hipMemoryTypeUnregistered) {
            (void)hipGetLastError();
            return err(CKR_E_INVALID, which ? "[ckr] gather destination is not device memory"
                                            : "[ckr] gather source is not device memory");
        }
        hipDeviceptr_t base = nullptr;
        size_t size = 0;
        if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) == hipSuccess && base) {
            const uintptr_t b = reinterpret_cast<uintptr_t>(base), q = reinterpret_cast<uintptr_t>(p);
            if (q < b || q - b > size || bytes > size - (q - b))
                return err(CKR_E_INVALID, which ? "[ckr] gather destination runs past its allocation"
                                                : "[ckr] strided source runs past its allocation");
        } else {
            (void)hipGetLastError();
        }
    }
    hipStream_t s = (hipStream_t)stream;
    const uint32_t grid = (uint32_t)std::min<uint64_t>((a.n + 255) / 256, 16384);
    switch (elem_size) {
        case 1: CKR_LAUNCH("gather_kernel", s, gather_kernel<uint8_t><<<grid, 256, 0, s>>>(static_cast<const uint8_t*>(d_src), static_cast<uint8_t*>(d_dst), a)); break;
        case 2: CKR_LAUNCH("gather_kernel", s, gather_kernel<uint16_t><<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(d_src), static_cast<uint16_t*>(d_dst), a)); break;
        case 4: CKR_LAUNCH("gather_kernel", s, gather_kernel<uint32_t><<<grid, 256, 0, s>>>(static_cast<const uint32_t*>(d_src), static_cast<uint32_t*>(d_dst), a)); break;
        default: CKR_LAUNCH("gather_kernel", s, gather_kernel<uint64_t><<<grid, 256, 0, s>>>(static_cast<const uint64_t*>(d_src), static_cast<uint64_t*>(d_dst), a)); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return err(CKR_E_HIP, std::string("[ckr] gather launch failed: ") + hipGetErrorString(e));
    return CKR_OK;
}

}  // extern "C"
