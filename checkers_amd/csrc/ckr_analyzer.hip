// checkers_amd/csrc/ckr_analyzer.hip — the statistics pass of TensorAnalyzer
// (src/TensorAnalyzer.cpp:64-198 compute_tensor_stats, :200-229
// tensor_stats_kernel, :281-290 the fingerprint) for any number of records in
// four launches: every record's blocks share one grid per pass.
//
//   pass 1  min, max and the fp64 sum of each block's share of its record
//   mid     per record: min, max, mean and the histogram scale
//   pass 2  per block: the 256-bin histogram (LDS, 16 copies, then added to
//           the record's histogram with global atomics) and the fp64 central
//           power sums 2..4
//   final   per record: moments, min/max and fingerprint
//
// Each block reads its share with 16-byte loads; the elements before the
// first 16-byte boundary of a record and those after its last whole vector
// are read one by one by the record's first block.  min/max are exact in any
// order; the histogram is bit-exact given them (the scale is rounded once
// from an fp64 quotient; double rounding of a float/float quotient through fp64
// is innocuous since 53 >= 2*24+2).  Sums: fp32 over the elements of one
// 16-byte vector (at most 16 terms, as the reference sums everything in fp32),
// fp64 beyond, reduced in a fixed order, so results do not depend on
// scheduling.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "ckr_internal.h"

namespace ckr {

namespace {

constexpr int kThreads = 256;
constexpr int kHistCopies = 16;  // 8, 16, 32 within 2%; 64 (a copy per lane) 35% slower
// Loads in flight per thread, and the grid: at most 256 workgroups per record,
// so that pass 2's closing global atomics (one per histogram bin and
// workgroup) stay few.  Measured on the cfg3 shard (4 records of 1G elements):
// 2048 workgroups per record and 2 loads in pass 2, 5.18 ms per call; 512,
// 4.95; 256, 4.70; 256 with 4 loads in pass 2, 4.61 (passes at 6.27 and 6.01
// TB/s); 128, 6.34 (pass 2 then lacks waves to hide its latency).
constexpr int kUnroll1 = 4, kUnroll2 = 4;
constexpr uint64_t kBytesPerBlock = 128 * 1024;
constexpr uint32_t kMaxBlocksPerRecord = 256;
constexpr uint32_t kDescPerStore = 40;

// A record as the kernels see it.
struct StatsDesc {
    const uint8_t* p;
    uint64_t n;          // elements
    uint32_t dt, bins;   // dtype tag; bins requested
    uint32_t blk0, nblk; // first block of the record in the grid, its block count
    uint32_t head;       // elements before the first 16-byte boundary
    uint32_t pad;
    uint32_t* hist;
    float *mom, *mm, *fp;
};

struct DescStoreArg {
    uint32_t n, off;
    StatsDesc d[kDescPerStore];
};

__global__ void stats_desc_store_kernel(DescStoreArg a, StatsDesc* __restrict__ out) {
    if (threadIdx.x < a.n) out[a.off + threadIdx.x] = a.d[threadIdx.x];
}

__device__ __forceinline__ float one(const uint8_t* p, uint64_t i, uint32_t dt) {
    switch (dt) {
        case CKR_F32: return reinterpret_cast<const float*>(p)[i];
        case CKR_BF16: return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
        case CKR_F16: return (float)reinterpret_cast<const _Float16*>(p)[i];
        case CKR_I8: return (float)reinterpret_cast<const int8_t*>(p)[i];
        default: return (float)reinterpret_cast<const int32_t*>(p)[i];
    }
}

// float → int32 as the hardware converts: out-of-range values (infinities
// included) saturate, NaN gives 0 — the clamp the bin index needs, in one
// instruction (the reference's int cast runs on the same conversion).
__device__ __forceinline__ int cvt_i32_sat(float t) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(t));
    return r;
}

// The 16 bytes v as DT's elements, each handed to f.
template <uint32_t DT, typename F>
__device__ __forceinline__ void unpack(const uint4 v, F&& f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    if constexpr (DT == CKR_F32) {
        for (int k = 0; k < 4; k++) f(__uint_as_float(w[k]));
    } else if constexpr (DT == CKR_I32) {
        for (int k = 0; k < 4; k++) f((float)(int32_t)w[k]);
    } else if constexpr (DT == CKR_BF16) {
        for (int k = 0; k < 4; k++) {
            f(__uint_as_float(w[k] << 16));
            f(__uint_as_float(w[k] & 0xFFFF0000u));
        }
    } else if constexpr (DT == CKR_F16) {
        for (int k = 0; k < 4; k++) {
            f((float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] & 0xFFFFu)));
            f((float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] >> 16)));
        }
    } else {  // int8
        for (int k = 0; k < 4; k++)
            for (int b = 0; b < 4; b++) f((float)(int8_t)(w[k] >> (8 * b)));
    }
}

// Calls f on every element of this block's share of record d: its 16-byte
// vectors (strided over the record's blocks), and, in the record's first block,
// the head and tail elements; g after each vector and after each of those
// elements.
template <uint32_t DT, int kUnroll, typename F, typename G>
__device__ __forceinline__ void for_share(const StatsDesc& d, uint32_t lb, F&& f, G&& g) {
    constexpr int ES = DT == CKR_F32 || DT == CKR_I32 ? 4 : DT == CKR_I8 ? 1 : 2;
    constexpr int VE = 16 / ES;
    const uint64_t head = d.head;
    const uint64_t nv = (d.n - head) / VE;
    const uint4* v = reinterpret_cast<const uint4*>(d.p + head * ES);
    const uint64_t stride = (uint64_t)d.nblk * kThreads;
    uint64_t i = (uint64_t)lb * kThreads + threadIdx.x;
    for (; i + (kUnroll - 1) * stride < nv; i += kUnroll * stride) {  // kUnroll loads in flight
        uint4 x[kUnroll];
        for (int k = 0; k < kUnroll; k++) x[k] = v[i + k * stride];
        for (int k = 0; k < kUnroll; k++) {
            unpack<DT>(x[k], f);
            g();
        }
    }
    for (; i < nv; i += stride) {
        unpack<DT>(v[i], f);
        g();
    }
    if (lb == 0) {
        const uint64_t tail0 = head + nv * VE;
        if (threadIdx.x < head) {
            f(one(d.p, threadIdx.x, DT));
            g();
        }
        if (tail0 + threadIdx.x < d.n) {
            f(one(d.p, tail0 + threadIdx.x, DT));
            g();
        }
    }
}

// Record of grid block b: the last record whose first block is <= b.
__device__ __forceinline__ uint32_t record_of(const StatsDesc* __restrict__ desc, uint32_t n, uint32_t b) {
    uint32_t lo = 0, hi = n - 1;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) >> 1;
        if (desc[mid].blk0 <= b) lo = mid; else hi = mid - 1;
    }
    return lo;
}

template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, T* sh, Op op) {
    sh[threadIdx.x] = v;
    __syncthreads();
    for (uint32_t s = kThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) sh[threadIdx.x] = op(sh[threadIdx.x], sh[threadIdx.x + s]);
        __syncthreads();
    }
    const T r = sh[0];
    __syncthreads();
    return r;
}

// The sum of one vector's elements in fp32 (at most 16 terms), then into the
// fp64 total.
template <uint32_t DT>
__device__ void pass1_share(const StatsDesc& d, uint32_t lb, float& mn, float& mx, double& sm) {
    float part = 0.f;
    for_share<DT, kUnroll1>(
        d, lb,
        [&](float x) {
            mn = fminf(mn, x);
            mx = fmaxf(mx, x);
            part += x;
        },
        [&] {
            sm += (double)part;
            part = 0.f;
        });
}

__global__ void __launch_bounds__(kThreads) stats_pass1_kernel(const StatsDesc* __restrict__ desc, uint32_t n_rec,
                                                               StatsPartial1* __restrict__ out) {
    __shared__ float shf[kThreads];
    __shared__ double shd[kThreads];
    const uint32_t r = record_of(desc, n_rec, blockIdx.x);
    const StatsDesc d = desc[r];
    const uint32_t lb = blockIdx.x - d.blk0;
    float mn = 1e37f, mx = -1e37f;  // the reference's initial values (TensorAnalyzer.cpp:97-98)
    double sm = 0.0;
    switch (d.dt) {
        case CKR_F32: pass1_share<CKR_F32>(d, lb, mn, mx, sm); break;
        case CKR_BF16: pass1_share<CKR_BF16>(d, lb, mn, mx, sm); break;
        case CKR_F16: pass1_share<CKR_F16>(d, lb, mn, mx, sm); break;
        case CKR_I8: pass1_share<CKR_I8>(d, lb, mn, mx, sm); break;
        default: pass1_share<CKR_I32>(d, lb, mn, mx, sm); break;
    }
    mn = block_reduce(mn, shf, [](float a, float b) { return fminf(a, b); });
    mx = block_reduce(mx, shf, [](float a, float b) { return fmaxf(a, b); });
    sm = block_reduce(sm, shd, [](double a, double b) { return a + b; });
    if (threadIdx.x == 0) out[blockIdx.x] = StatsPartial1{mn, mx, sm};
}

__global__ void __launch_bounds__(kThreads) stats_mid_kernel(const StatsDesc* __restrict__ desc,
                                                             const StatsPartial1* __restrict__ p1,
                                                             StatsParams* __restrict__ prm) {
    __shared__ float shf[kThreads];
    __shared__ double shd[kThreads];
    const StatsDesc d = desc[blockIdx.x];
    float mn = 1e37f, mx = -1e37f;
    double sm = 0.0;
    for (uint32_t b = threadIdx.x; b < d.nblk; b += kThreads) {
        const StatsPartial1 q = p1[d.blk0 + b];
        mn = fminf(mn, q.mn);
        mx = fmaxf(mx, q.mx);
        sm += q.sum;
    }
    mn = block_reduce(mn, shf, [](float a, float b) { return fminf(a, b); });
    mx = block_reduce(mx, shf, [](float a, float b) { return fmaxf(a, b); });
    sm = block_reduce(sm, shd, [](double a, double b) { return a + b; });
    const uint32_t bins = d.bins < 256u ? d.bins : 256u;  // TensorAnalyzer.cpp:73
    if (threadIdx.x < bins && d.hist) d.hist[threadIdx.x] = 0;  // pass 2 adds into it
    if (threadIdx.x == 0) {
        const float range = mx - mn;
        StatsParams q;
        q.smin = mn;
        q.smax = mx;
        q.mean = (float)(sm / (double)d.n);
        q.use_range = range > 1e-9f ? 1u : 0u;
        q.scale = q.use_range ? (float)((double)((float)bins - 1.0f) / (double)range) : 0.0f;
        q.bins = bins;
        q.pad[0] = q.pad[1] = 0;
        prm[blockIdx.x] = q;
    }
}

// Central powers as the reference forms them (float d = x - mean), summed in
// fp32 over one vector's elements, then into fp64 totals.
template <uint32_t DT>
__device__ void pass2_share(const StatsDesc& d, uint32_t lb, const StatsParams& q, uint32_t* sh, double& a2,
                            double& a3, double& a4) {
    const uint32_t c = threadIdx.x & (kHistCopies - 1);
    const float mean = q.mean;
    float p2 = 0.f, p3 = 0.f, p4 = 0.f;
    for_share<DT, kUnroll2>(
        d, lb,
        [&](float x) {
            if (q.bins > 0) {
                int b = 0;
                if (q.use_range) {  // TensorAnalyzer.cpp:150-160
                    const float t = __fmul_rn(__fsub_rn(x, q.smin), q.scale);
                    b = max(0, min(cvt_i32_sat(t), (int)q.bins - 1));
                }
                atomicAdd(&sh[b * kHistCopies + c], 1u);
            }
            const float dd = __fsub_rn(x, mean), d2 = __fmul_rn(dd, dd);
            p2 += d2;
            p3 = fmaf(d2, dd, p3);
            p4 = fmaf(d2, d2, p4);
        },
        [&] {
            a2 += (double)p2;
            a3 += (double)p3;
            a4 += (double)p4;
            p2 = p3 = p4 = 0.f;
        });
}

__global__ void __launch_bounds__(kThreads) stats_pass2_kernel(const StatsDesc* __restrict__ desc, uint32_t n_rec,
                                                               const StatsParams* __restrict__ prm,
                                                               StatsPartial2* __restrict__ out) {
    __shared__ uint32_t sh[256 * kHistCopies];
    __shared__ double shd[kThreads];
    for (uint32_t i = threadIdx.x; i < 256 * kHistCopies; i += kThreads) sh[i] = 0;
    __syncthreads();
    const uint32_t r = record_of(desc, n_rec, blockIdx.x);
    const StatsDesc d = desc[r];
    const StatsParams q = prm[r];
    const uint32_t lb = blockIdx.x - d.blk0;
    double a2 = 0, a3 = 0, a4 = 0;
    switch (d.dt) {
        case CKR_F32: pass2_share<CKR_F32>(d, lb, q, sh, a2, a3, a4); break;
        case CKR_BF16: pass2_share<CKR_BF16>(d, lb, q, sh, a2, a3, a4); break;
        case CKR_F16: pass2_share<CKR_F16>(d, lb, q, sh, a2, a3, a4); break;
        case CKR_I8: pass2_share<CKR_I8>(d, lb, q, sh, a2, a3, a4); break;
        default: pass2_share<CKR_I32>(d, lb, q, sh, a2, a3, a4); break;
    }
    const auto add = [](double a, double b) { return a + b; };
    a2 = block_reduce(a2, shd, add);
    a3 = block_reduce(a3, shd, add);
    a4 = block_reduce(a4, shd, add);
    if (threadIdx.x < q.bins && d.hist) {
        uint32_t hs = 0;
        for (int k = 0; k < kHistCopies; k++) hs += sh[threadIdx.x * kHistCopies + k];
        if (hs) atomicAdd(&d.hist[threadIdx.x], hs);
    }
    if (threadIdx.x == 0) out[blockIdx.x] = StatsPartial2{a2, a3, a4, 0.0};
}

__global__ void __launch_bounds__(kThreads) stats_final_kernel(const StatsDesc* __restrict__ desc,
                                                               const StatsPartial2* __restrict__ p2,
                                                               const StatsParams* __restrict__ prm) {
    __shared__ double shd[kThreads];
    const StatsDesc d = desc[blockIdx.x];
    const StatsParams q = prm[blockIdx.x];
    const uint32_t t = threadIdx.x;
    double m2 = 0, m3 = 0, m4 = 0;
    for (uint32_t b = t; b < d.nblk; b += kThreads) {
        const StatsPartial2 v = p2[d.blk0 + b];
        m2 += v.m2;
        m3 += v.m3;
        m4 += v.m4;
    }
    const auto add = [](double a, double b) { return a + b; };
    m2 = block_reduce(m2, shd, add);
    m3 = block_reduce(m3, shd, add);
    m4 = block_reduce(m4, shd, add);
    if (t == 0) {  // TensorAnalyzer.cpp:170-198, fingerprint :281-290
        const float M2 = (float)(m2 / (double)d.n), M3 = (float)(m3 / (double)d.n), M4 = (float)(m4 / (double)d.n);
        const float var = M2;
        float skew = 0.f, kurt = 0.f;
        if (var > 1e-9f) {
            const float sd = sqrtf(var);
            skew = M3 / (var * sd);
            kurt = M4 / (var * var);
        }
        if (d.mom) { d.mom[0] = q.mean; d.mom[1] = var; d.mom[2] = skew; d.mom[3] = kurt; }
        if (d.mm) { d.mm[0] = q.smin; d.mm[1] = q.smax; }
        if (d.fp) { d.fp[0] = q.mean; d.fp[1] = var; d.fp[2] = skew; d.fp[3] = kurt; d.fp[4] = q.smax - q.smin; }
    }
}

bool analyzable(const ckr_stats_record& r) {
    return r.d_ptr && r.num_elements && (r.data_type == CKR_F32 || r.data_type == CKR_BF16 ||
                                         r.data_type == CKR_F16 || r.data_type == CKR_I8 || r.data_type == CKR_I32);
}

uint32_t blocks_for(const ckr_stats_record& r) {
    const uint64_t bytes = r.num_elements * (uint64_t)ckr_element_size((int)r.data_type);
    return (uint32_t)std::min<uint64_t>(std::max<uint64_t>((bytes + kBytesPerBlock - 1) / kBytesPerBlock, 1),
                                        kMaxBlocksPerRecord);
}

uint64_t al(uint64_t v) { return (v + 255) / 256 * 256; }

struct Layout {
    uint64_t desc, p1, prm, p2, total;
};
Layout layout(uint64_t n_rec, uint64_t n_blk) {
    Layout L;
    L.desc = 0;
    L.p1 = L.desc + al(n_rec * sizeof(StatsDesc));
    L.prm = L.p1 + al(n_blk * sizeof(StatsPartial1));
    L.p2 = L.prm + al(n_rec * sizeof(StatsParams));
    L.total = L.p2 + al(n_blk * sizeof(StatsPartial2));
    return L;
}

}  // namespace

uint64_t analyze_workspace_bytes(const ckr_stats_record* recs, uint64_t n) {
    uint64_t nr = 0, nb = 0;
    for (uint64_t i = 0; i < n; i++)
        if (analyzable(recs[i])) {
            nr++;
            nb += blocks_for(recs[i]);
        }
    return nr ? layout(nr, nb).total : 0;
}

hipError_t launch_analyze(const ckr_stats_record* recs, uint64_t n, void* ws, hipStream_t s) {
    std::vector<StatsDesc> d;
    uint64_t nb = 0;
    for (uint64_t i = 0; i < n; i++) {
        const ckr_stats_record& r = recs[i];
        if (!analyzable(r)) continue;  // TensorAnalyzer.cpp:68, tensor_stats_kernel's default branch
        StatsDesc x{};
        x.p = static_cast<const uint8_t*>(r.d_ptr);
        x.n = r.num_elements;
        x.dt = r.data_type;
        x.bins = r.histogram_bins;
        x.blk0 = (uint32_t)nb;
        x.nblk = blocks_for(r);
        const uint64_t es = (uint64_t)ckr_element_size((int)r.data_type);
        const uint64_t mis = reinterpret_cast<uintptr_t>(r.d_ptr) & 15u;
        x.head = (uint32_t)std::min<uint64_t>(mis ? (16 - mis) / es : 0, r.num_elements);
        x.hist = r.d_histogram;
        x.mom = r.d_raw_moments;
        x.mm = r.d_minmax;
        x.fp = r.d_fingerprint;
        nb += x.nblk;
        d.push_back(x);
    }
    if (d.empty()) return hipSuccess;
    const Layout L = layout(d.size(), nb);
    uint8_t* w = static_cast<uint8_t*>(ws);
    auto* desc = reinterpret_cast<StatsDesc*>(w + L.desc);
    auto* p1 = reinterpret_cast<StatsPartial1*>(w + L.p1);
    auto* prm = reinterpret_cast<StatsParams*>(w + L.prm);
    auto* p2 = reinterpret_cast<StatsPartial2*>(w + L.p2);
    // descriptors travel as kernel arguments: no host buffer outlives the call
    for (uint32_t off = 0; off < d.size(); off += kDescPerStore) {
        DescStoreArg a{};
        a.off = off;
        a.n = (uint32_t)std::min<uint64_t>(kDescPerStore, d.size() - off);
        std::copy(d.begin() + off, d.begin() + off + a.n, a.d);
        CKR_LAUNCH("stats_desc_store_kernel", s, stats_desc_store_kernel<<<1, 64, 0, s>>>(a, desc));
    }
    const uint32_t nr = (uint32_t)d.size();
    CKR_LAUNCH("stats_pass1_kernel", s, stats_pass1_kernel<<<(uint32_t)nb, kThreads, 0, s>>>(desc, nr, p1));
    CKR_LAUNCH("stats_mid_kernel", s, stats_mid_kernel<<<nr, kThreads, 0, s>>>(desc, p1, prm));
    CKR_LAUNCH("stats_pass2_kernel", s, stats_pass2_kernel<<<(uint32_t)nb, kThreads, 0, s>>>(desc, nr, prm, p2));
    CKR_LAUNCH("stats_final_kernel", s, stats_final_kernel<<<nr, kThreads, 0, s>>>(desc, p2, prm));
    return hipGetLastError();
}

}  // namespace ckr
