// oracle/ckr_oracle.cpp — CPU restatement of the reference's checkpoint-compression
// hot path.  TEST INFRASTRUCTURE ONLY: it is the checker for the HIP library, and
// the CPU baseline timed beside it.  Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg load it; the product never does.
//
// Every function follows the cited reference code (paths relative to the
// reference tree).  How each one is pinned (closed forms, brute force,
// invariants) is listed in tests/test_oracle.py; nothing here is pinned by
// re-typing its own formula.
//
// Built by oracle/Makefile with g++ (libstdc++ std::sort is required: the table
// tie order depends on it, see normalize_histogram below).

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <unordered_map>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

extern "C" {

// ---------------------------------------------------------------- constants
// include/checkers/ANSCompressor.hpp:51-55
static const uint32_t OC_SCALE_BITS = 12;
static const uint32_t OC_M = 1u << OC_SCALE_BITS;
static const uint32_t OC_L = 1u << 23;
static const uint32_t OC_NORM_BASE = (OC_L >> OC_SCALE_BITS) << 8;
static const uint32_t OC_LANES = 256;

struct oc_header { uint32_t final_state, byte_count, buf_offset, pad; };  // ANSCompressor.hpp:79-84

// include/checkers/ANSCompressor.hpp:64-74
struct alignas(64) oc_table {
    uint32_t norm_freq[256];
    uint32_t cum_freq[257];
    uint32_t x_max[256];
    uint8_t decode_sym[4096];
    uint32_t decode_freq[4096];
    uint32_t decode_cum[4096];
};
static_assert(sizeof(oc_table) == 40000, "ANSFreqTable layout");
static_assert(sizeof(oc_header) == 16, "ANSStreamHeader layout");

// include/checkers/TensorResource.hpp:39-48
int oc_element_size(int dtype) {
    switch (dtype) {
        case 0: return 4; case 1: return 2; case 2: return 2; case 3: return 1; case 4: return 4;
        default: return 0;
    }
}

// src/ANSCompressor.cpp:955-967 (fp16/bf16: 1 low byte, fp32: 2 low bytes, others none)
int oc_sidecar_per_elem(int dtype) {
    switch (dtype) {
        case 0: return 2; case 1: return 1; case 2: return 1;
        default: return 0;
    }
}

// ---------------------------------------------------------------- byte-plane split
// src/ANSCompressor.cpp:258-279: masked = element with its low `spe` bytes zeroed,
// sidecar[i*spe + j] = src[i*es + j].  Returns spe (0: unsupported dtype, nothing written).
int oc_extract_mantissa(const uint8_t* src, uint64_t n, int dtype, uint8_t* masked, uint8_t* sidecar) {
    const int es = oc_element_size(dtype), spe = oc_sidecar_per_elem(dtype);
    if (spe == 0) return 0;
    for (uint64_t i = 0; i < n; i++) {
        for (int j = 0; j < es; j++) masked[i * es + j] = (j < spe) ? 0 : src[i * es + j];
        for (int j = 0; j < spe; j++) sidecar[i * spe + j] = src[i * es + j];
    }
    return spe;
}

// src/ANSCompressor.cpp:109-126 — plain count of every byte value.
void oc_byte_hist(const uint8_t* data, uint64_t n, uint32_t* hist) {
    for (int i = 0; i < 256; i++) hist[i] = 0;
    for (uint64_t i = 0; i < n; i++) hist[data[i]]++;
}

// The same two steps on n_threads host threads (OpenMP over element / byte
// ranges; per-thread counts summed), for the CPU baseline's threaded leg.
// Results equal the single-thread functions' (u32 counts wrap alike).
int oc_extract_mantissa_mt(const uint8_t* src, uint64_t n, int dtype, uint8_t* masked, uint8_t* sidecar,
                           int n_threads) {
    const int es = oc_element_size(dtype), spe = oc_sidecar_per_elem(dtype);
    if (spe == 0) return 0;
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t i = 0; i < (int64_t)n; i++) {
        for (int j = 0; j < es; j++) masked[i * es + j] = (j < spe) ? 0 : src[i * es + j];
        for (int j = 0; j < spe; j++) sidecar[i * spe + j] = src[i * es + j];
    }
    return spe;
}

void oc_byte_hist_mt(const uint8_t* data, uint64_t n, uint32_t* hist, int n_threads) {
    for (int i = 0; i < 256; i++) hist[i] = 0;
#pragma omp parallel num_threads(n_threads)
    {
        uint32_t h[256] = {};
#pragma omp for schedule(static)
        for (int64_t i = 0; i < (int64_t)n; i++) h[data[i]]++;
#pragma omp critical
        for (int i = 0; i < 256; i++) hist[i] += h[i];
    }
}

// ---------------------------------------------------------------- table
// src/ANSCompressor.cpp:416-503, step by step.  The decode arrays are written
// only for slots < 4096: the reference writes past them when the table sum
// exceeds 4096 (its single decrement pass, :477-482); the returned value is the
// table sum so that callers can see that case.
uint32_t oc_normalize_histogram(const uint32_t* h, int ensure_full_alphabet, oc_table* t) {
    std::memset(t, 0, sizeof(*t));
    uint64_t total = 0;
    int n_distinct = 0;
    for (int i = 0; i < 256; i++) { total += h[i]; n_distinct += h[i] > 0; }
    const int effective = ensure_full_alphabet ? 256 : n_distinct;
    if (effective == 0) {  // :432-442
        t->norm_freq[0] = OC_M;
        for (int i = 1; i <= 256; i++) t->cum_freq[i] = OC_M;
        t->x_max[0] = OC_NORM_BASE * OC_M;
        for (uint32_t j = 0; j < OC_M; j++) { t->decode_sym[j] = 0; t->decode_freq[j] = OC_M; t->decode_cum[j] = 0; }
        return OC_M;
    }
    uint32_t norm[256] = {};
    uint32_t assigned = 0;
    for (int i = 0; i < 256; i++) {  // :448-456
        if (!ensure_full_alphabet && h[i] == 0) continue;
        uint32_t slots = total > 0 ? (uint32_t)((uint64_t)std::max(h[i], 1u) * OC_M / total) : 0u;
        if (slots == 0) slots = 1;
        norm[i] = slots;
        assigned += slots;
    }
    struct SF { int sym; double frac; };
    std::vector<SF> fracs;
    fracs.reserve(256);
    for (int i = 0; i < 256; i++) {  // :462-468
        if (norm[i] == 0) continue;
        double exact = total > 0 ? ((double)std::max(h[i], 1u) * OC_M / (double)total) : 1.0;
        fracs.push_back({i, exact - (double)(int)exact});
    }
    // :469-471 — libstdc++ introsort; ties among equal fractions keep whatever
    // order this exact call produces, which is why the library must be the same.
    std::sort(fracs.begin(), fracs.end(), [](const SF& a, const SF& b) { return a.frac > b.frac; });
    if (assigned < OC_M) {  // :473-476
        uint32_t rem = OC_M - assigned;
        for (size_t k = 0; k < fracs.size() && rem; k++, rem--) norm[fracs[k].sym]++;
    } else if (assigned > OC_M) {  // :477-482 (one pass only)
        uint32_t rem = assigned - OC_M;
        for (int k = (int)fracs.size() - 1; k >= 0 && rem; k--)
            if (norm[fracs[k].sym] > 1) { norm[fracs[k].sym]--; rem--; }
    }
    for (int i = 0; i < 256; i++) t->norm_freq[i] = norm[i];  // :486-500
    t->cum_freq[0] = 0;
    for (int i = 0; i < 256; i++) t->cum_freq[i + 1] = t->cum_freq[i] + t->norm_freq[i];
    for (int s = 0; s < 256; s++) {
        if (t->norm_freq[s] == 0) { t->x_max[s] = 0; continue; }
        t->x_max[s] = OC_NORM_BASE * t->norm_freq[s];
        for (uint32_t j = t->cum_freq[s]; j < t->cum_freq[s + 1] && j < OC_M; j++) {
            t->decode_sym[j] = (uint8_t)s;
            t->decode_freq[j] = t->norm_freq[s];
            t->decode_cum[j] = t->cum_freq[s];
        }
    }
    return t->cum_freq[256];
}

// ---------------------------------------------------------------- encode
// One lane of rans_encode_kernel (src/ANSCompressor.cpp:154-211), literal: the
// unit's bytes d[0..n), lane `tid`, output written backward from region_end,
// region of max_chunk = 2*ceil(n/256) bytes.  Returns the number of bytes
// written; *final_state receives the state.
static uint32_t encode_lane(const uint8_t* d, uint64_t n, const oc_table* t, uint32_t tid,
                            uint8_t* region_start, uint64_t max_chunk, uint32_t* final_state) {
    const uint64_t count = n > tid ? (n - tid + OC_LANES - 1) / OC_LANES : 0;
    uint8_t* const region_end = region_start + max_chunk;
    uint8_t* w = region_end;
    uint32_t state = OC_L;
    for (uint64_t k = count; k-- > 0;) {
        const uint8_t sym = d[tid + k * OC_LANES];
        const uint32_t freq = t->norm_freq[sym], cum = t->cum_freq[sym], xm = t->x_max[sym];
        if (freq == 0) {  // :185-192 escape: raw byte, no state update
            if (w > region_start) *--w = sym;
            continue;
        }
        while (state >= xm) {  // :195-199
            if (w <= region_start) { w = region_start; break; }
            *--w = (uint8_t)(state & 0xFFu);
            state >>= 8;
        }
        state = ((state / freq) << OC_SCALE_BITS) + cum + (state % freq);  // :202
    }
    *final_state = state;
    return (uint32_t)(region_end - w);
}

// Encode one unit of n bytes: the 256 lanes, then the host prefix sum and
// compaction of compress_tensor (src/ANSCompressor.cpp:641-691), then the
// passthrough rule (:694-713: packed size >= n ⇒ store the bytes as they are,
// headers zeroed except headers[0].byte_count = n).  Writes to out[0..) and
// returns the unit's data size.
static uint64_t encode_unit(const uint8_t* d, uint64_t n, const oc_table* t, uint8_t* out,
                            oc_header* hdr, std::vector<uint8_t>& scratch) {
    const uint64_t max_chunk = ((n + OC_LANES - 1) / OC_LANES) * 2;  // :590
    scratch.resize(max_chunk * OC_LANES);
    uint64_t off = 0;
    uint32_t cnt[256], fs[256];
    for (uint32_t l = 0; l < OC_LANES; l++)
        cnt[l] = encode_lane(d, n, t, l, scratch.data() + l * max_chunk, max_chunk, &fs[l]);
    for (uint32_t l = 0; l < OC_LANES; l++) off += cnt[l];
    if (n > 0 && off >= n) {
        std::memcpy(out, d, n);
        std::memset(hdr, 0, OC_LANES * sizeof(oc_header));
        hdr[0].byte_count = (uint32_t)n;
        return n;
    }
    off = 0;
    for (uint32_t l = 0; l < OC_LANES; l++) {
        std::memcpy(out + off, scratch.data() + l * max_chunk + (max_chunk - cnt[l]), cnt[l]);
        hdr[l].final_state = fs[l];
        hdr[l].byte_count = cnt[l];
        hdr[l].buf_offset = (uint32_t)off;
        hdr[l].pad = 0;
        off += cnt[l];
    }
    return off;
}

uint64_t oc_num_units(uint64_t n_b, uint64_t unit) {
    if (n_b == 0) return 0;
    if (unit == 0 || unit >= n_b) return 1;
    return (n_b + unit - 1) / unit;
}

// Chunked encode of a masked byte stream: unit after unit (unit == 0 or
// unit >= n_b: one unit, the reference's whole-tensor layout).  out must hold
// n_b + 2*256*... — callers size it as n_b * 2 + 512 per unit.
// Returns C (total data bytes).  unit_off has n_units + 1 entries.
uint64_t oc_encode(const uint8_t* masked, uint64_t n_b, const oc_table* t, uint64_t unit,
                   uint8_t* out, oc_header* hdrs, uint64_t* unit_off, int n_threads) {
    const uint64_t nu = oc_num_units(n_b, unit);
    const uint64_t U = (nu <= 1) ? n_b : unit;
    std::vector<uint64_t> sizes(nu);
    // Units are independent; with n_threads > 1 they are coded in parallel into
    // per-unit staging and packed afterwards (the CPU baseline's OpenMP variant).
    if (n_threads <= 1 || nu <= 1) {
        std::vector<uint8_t> scratch;
        uint64_t off = 0;
        for (uint64_t u = 0; u < nu; u++) {
            const uint64_t len = std::min<uint64_t>(U, n_b - u * U);
            unit_off[u] = off;
            off += encode_unit(masked + u * U, len, t, out + off, hdrs + u * OC_LANES, scratch);
        }
        unit_off[nu] = off;
        return off;
    }
    std::vector<std::vector<uint8_t>> staged(nu);
#ifdef _OPENMP
#pragma omp parallel num_threads(n_threads)
#endif
    {
        std::vector<uint8_t> scratch;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
        for (int64_t u = 0; u < (int64_t)nu; u++) {
            const uint64_t len = std::min<uint64_t>(U, n_b - u * U);
            staged[u].resize(len);
            sizes[u] = encode_unit(masked + u * U, len, t, staged[u].data(), hdrs + u * OC_LANES, scratch);
        }
    }
    uint64_t off = 0;
    for (uint64_t u = 0; u < nu; u++) {
        unit_off[u] = off;
        std::memcpy(out + off, staged[u].data(), sizes[u]);
        off += sizes[u];
    }
    unit_off[nu] = off;
    return off;
}

// ---------------------------------------------------------------- decode
// The decoder the encoder implies (the reference has none): for lane t,
// x = final_state, read forward; slot = x & 4095; s = decode_sym[slot];
// x = f*(x>>12) + slot - cum; refill bytes while x < 2^23.  Checks: the lane
// ends in state 2^23 and has read exactly byte_count bytes.  Returns the number
// of lanes that fail these checks (0 for a valid stream).  Requires a table
// with sum(norm_freq) == 4096.
uint64_t oc_decode(const uint8_t* data, const oc_header* hdrs, const uint64_t* unit_off,
                   const oc_table* t, uint64_t n_b, uint64_t unit, uint8_t* masked_out) {
    const uint64_t nu = oc_num_units(n_b, unit);
    const uint64_t U = (nu <= 1) ? n_b : unit;
    uint64_t bad = 0;
    for (uint64_t u = 0; u < nu; u++) {
        const uint64_t len = std::min<uint64_t>(U, n_b - u * U);
        const uint8_t* ud = data + unit_off[u];
        const oc_header* h = hdrs + u * OC_LANES;
        uint8_t* o = masked_out + u * U;
        bool raw = h[0].byte_count == (uint32_t)len;  // writer's raw test, ANSCompressor.cpp:787-789
        for (uint32_t l = 1; l < OC_LANES && raw; l++) raw = h[l].byte_count == 0;
        if (raw && unit_off[u + 1] - unit_off[u] == len) { std::memcpy(o, ud, len); continue; }
        for (uint32_t l = 0; l < OC_LANES; l++) {
            const uint64_t count = len > l ? (len - l + OC_LANES - 1) / OC_LANES : 0;
            uint32_t x = h[l].final_state;
            const uint8_t* p = ud + h[l].buf_offset;
            const uint8_t* end = p + h[l].byte_count;
            for (uint64_t k = 0; k < count; k++) {
                const uint32_t slot = x & (OC_M - 1);
                const uint8_t s = t->decode_sym[slot];
                o[l + k * OC_LANES] = s;
                x = t->norm_freq[s] * (x >> OC_SCALE_BITS) + slot - t->cum_freq[s];
                while (x < OC_L && p < end) x = (x << 8) | *p++;
            }
            if (x != OC_L || p != end) bad++;
        }
    }
    return bad;
}

// Sidecar merge: original = masked | sidecar (ANSCompressor.hpp:165-171).
void oc_merge_sidecar(const uint8_t* masked, const uint8_t* sidecar, uint64_t n, int dtype, uint8_t* dst) {
    const int es = oc_element_size(dtype), spe = oc_sidecar_per_elem(dtype);
    for (uint64_t i = 0; i < n; i++)
        for (int j = 0; j < es; j++)
            dst[i * es + j] = (j < spe) ? sidecar[i * spe + j] : masked[i * es + j];
}

// ---------------------------------------------------------------- analyzer
static inline float half_to_float(uint16_t h) {  // exact IEEE half → float
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = s;
        else {  // subnormal: value m * 2^-24, exact in float
            float f = (float)m * 5.9604644775390625e-08f;
            std::memcpy(&bits, &f, 4);
            bits |= s;
        }
    } else if (e == 31) bits = s | 0x7F800000u | (m << 13);
    else bits = s | ((e + 112) << 23) | (m << 13);
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}
static inline float load_as_float(const uint8_t* p, uint64_t i, int dtype) {
    switch (dtype) {
        case 0: { float f; std::memcpy(&f, p + 4 * i, 4); return f; }
        case 1: { uint16_t b; std::memcpy(&b, p + 2 * i, 2); uint32_t u = (uint32_t)b << 16; float f; std::memcpy(&f, &u, 4); return f; }
        case 2: { uint16_t b; std::memcpy(&b, p + 2 * i, 2); return half_to_float(b); }
        case 3: return (float)(int8_t)p[i];
        case 4: { int32_t v; std::memcpy(&v, p + 4 * i, 4); return (float)v; }
        default: return 0.f;
    }
}
// float→int conversion as the GPU's v_cvt_i32_f32 does it (NaN → 0, saturating);
// the reference's static_cast<int> leaves NaN undefined in C++.
static inline int cvt_i32_sat(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (-2147483647 - 1);
    return (int)v;
}

// compute_tensor_stats<T> (src/TensorAnalyzer.cpp:64-198) in the reference's own
// order (thread t handles t, t+256, …; LDS tree 128→1), fp32 throughout.
// Outputs hist[min(bins,256)], moments[4] (mean, var, skew, kurt), minmax[2];
// moments64[4] receives the same four statistics in fp64 (two-pass, exact-ish)
// for tolerance checks.
void oc_tensor_stats(const uint8_t* data, uint64_t N, int dtype, uint32_t bins_in,
                     uint32_t* hist, float* moments, float* minmax, double* moments64) {
    const uint32_t bins = bins_in < 256u ? bins_in : 256u;
    if (N == 0) return;
    float rmin[256], rmax[256], rsum[256];
    for (int tid = 0; tid < 256; tid++) {
        float lmin = 1e37f, lmax = -1e37f, lsum = 0.0f;
        for (uint64_t i = tid; i < N; i += 256) {
            float x = load_as_float(data, i, dtype);
            lmin = std::fmin(lmin, x);
            lmax = std::fmax(lmax, x);
            lsum += x;
        }
        rmin[tid] = lmin; rmax[tid] = lmax; rsum[tid] = lsum;
    }
    for (int s = 128; s > 0; s >>= 1)
        for (int tid = 0; tid < s; tid++) {
            rmin[tid] = std::fmin(rmin[tid], rmin[tid + s]);
            rmax[tid] = std::fmax(rmax[tid], rmax[tid + s]);
            rsum[tid] += rsum[tid + s];
        }
    const float smin = rmin[0], smax = rmax[0], mean = rsum[0] / (float)N;
    const float range = smax - smin;
    const float scale = (range > 1e-9f) ? ((float)bins - 1.0f) / range : 0.0f;
    std::vector<uint32_t> hh(256, 0);
    float m2[256], m3[256], m4[256];
    for (int tid = 0; tid < 256; tid++) {
        float a2 = 0, a3 = 0, a4 = 0;
        for (uint64_t i = tid; i < N; i += 256) {
            float x = load_as_float(data, i, dtype);
            if (range > 1e-9f) {
                int b = cvt_i32_sat((x - smin) * scale);
                b = std::max(0, std::min(b, (int)(bins - 1)));
                hh[b]++;
            } else if (bins > 0) {
                hh[0]++;
            }
            float d = x - mean, d2 = d * d;
            a2 += d2; a3 += d2 * d; a4 += d2 * d2;
        }
        m2[tid] = a2; m3[tid] = a3; m4[tid] = a4;
    }
    for (int s = 128; s > 0; s >>= 1)
        for (int tid = 0; tid < s; tid++) { m2[tid] += m2[tid + s]; m3[tid] += m3[tid + s]; m4[tid] += m4[tid + s]; }
    if (hist) for (uint32_t b = 0; b < bins; b++) hist[b] = hh[b];
    const float M2 = m2[0] / (float)N, M3 = m3[0] / (float)N, M4 = m4[0] / (float)N;
    float var = M2, skew = 0.f, kurt = 0.f;
    if (var > 1e-9f) { float sd = std::sqrt(var); skew = M3 / (var * sd); kurt = M4 / (var * var); }
    if (moments) { moments[0] = mean; moments[1] = var; moments[2] = skew; moments[3] = kurt; }
    if (minmax) { minmax[0] = smin; minmax[1] = smax; }
    if (moments64) {
        double s = 0;
        for (uint64_t i = 0; i < N; i++) s += (double)load_as_float(data, i, dtype);
        const double mu = s / (double)N;
        double c2 = 0, c3 = 0, c4 = 0;
        for (uint64_t i = 0; i < N; i++) {
            double d = (double)load_as_float(data, i, dtype) - mu, d2 = d * d;
            c2 += d2; c3 += d2 * d; c4 += d2 * d2;
        }
        c2 /= (double)N; c3 /= (double)N; c4 /= (double)N;
        moments64[0] = mu; moments64[1] = c2;
        moments64[2] = c2 > 0 ? c3 / (c2 * std::sqrt(c2)) : 0.0;
        moments64[3] = c2 > 0 ? c4 / (c2 * c2) : 0.0;
    }
}

// ---------------------------------------------------------------- prefix-mask repair
// src/tensor_group_prefix_mask_repair.cpp: build_masked_sequence (:328-353),
// find_best_pair (:376-405), apply_rule (:407-426), build_shared_grammar
// (:428-457), apply_existing_grammar (:459-467).
//
// The pair counts live in a libstdc++ std::unordered_map with the same key
// hash (lhs ^ (rhs + 0x9e3779b97f4a7c15 + (lhs << 6) + (lhs >> 2)), identity
// std::hash<uint64_t>) and the same reserve(size) call per round, so the
// iteration order that breaks ties between equally frequent pairs is the
// library's own.  A symbol is a uint64_t: masked words keep their bit
// positions, rule i is 2^63 + i.

struct oc_pair { uint64_t l, r; bool operator==(const oc_pair& o) const { return l == o.l && r == o.r; } };
struct oc_pair_hash {
    size_t operator()(const oc_pair& k) const {
        const size_t a = std::hash<uint64_t>{}(k.l), b = std::hash<uint64_t>{}(k.r);
        return a ^ (b + 0x9e3779b97f4a7c15ull + (a << 6) + (a >> 2));
    }
};

// Masked word sequence of n little-endian words of `storage_bytes` (2 or 4)
// with the low `masked_bits` bits cleared.
static std::vector<uint64_t> repair_masked_words(const uint8_t* raw, uint64_t n, int storage_bytes,
                                                 uint32_t masked_bits) {
    const uint64_t mask = masked_bits ? ((uint64_t)1 << masked_bits) - 1 : 0;
    std::vector<uint64_t> w(n);
    for (uint64_t i = 0; i < n; i++) {
        uint64_t v = 0;
        for (int b = 0; b < storage_bytes; b++) v |= (uint64_t)raw[i * storage_bytes + b] << (8 * b);
        w[i] = v & ~mask;
    }
    return w;
}

// One greedy left-to-right pass replacing non-overlapping (l, r) by `sym`.
static uint64_t repair_apply_rule(std::vector<uint64_t>& t, uint64_t l, uint64_t r, uint64_t sym) {
    uint64_t o = 0, rep = 0;
    for (uint64_t i = 0; i < t.size();) {
        if (i + 1 < t.size() && t[i] == l && t[i + 1] == r) { t[o++] = sym; i += 2; rep++; }
        else t[o++] = t[i++];
    }
    t.resize(o);
    return rep;
}

// Bucket count std::unordered_map picks for reserve(n) (for tests of the
// product's own computation of it).
uint64_t oc_repair_bucket_count(uint64_t n) {
    std::unordered_map<oc_pair, size_t, oc_pair_hash> m;
    m.reserve(n);
    return m.bucket_count();
}

// Rounds of the last oc_repair_build whose largest pair count was shared by
// more than one pair (the rounds in which the map's iteration order decides).
static uint32_t g_tied_rounds = 0;
uint32_t oc_repair_last_tied_rounds() { return g_tied_rounds; }

// build_shared_grammar on the masked sequence.  rules[4*i..] = {replacement,
// lhs, rhs, frequency}.  Returns the rule count; *out_len the compressed
// length, *max_pair the largest pair count seen in any round.  seq_out (n
// entries, may be NULL) receives the compressed sequence.
uint32_t oc_repair_build(const uint8_t* raw, uint64_t n, int storage_bytes, uint32_t masked_bits,
                         uint32_t max_rules, uint64_t* rules, uint64_t* out_len, uint64_t* max_pair,
                         uint64_t* seq_out) {
    std::vector<uint64_t> t = repair_masked_words(raw, n, storage_bytes, masked_bits);
    uint64_t next = (uint64_t)1 << 63, maxf = 0;
    uint32_t nr = 0;
    g_tied_rounds = 0;
    for (uint32_t ri = 0; ri < max_rules; ri++) {
        if (t.size() < 2) break;
        std::unordered_map<oc_pair, size_t, oc_pair_hash> counts;
        counts.reserve(t.size());
        for (size_t i = 0; i + 1 < t.size(); i++) ++counts[{t[i], t[i + 1]}];
        size_t best = 0;
        oc_pair bp{0, 0};
        for (const auto& kv : counts) {
            maxf = std::max<uint64_t>(maxf, kv.second);
            if (kv.second > best) { best = kv.second; bp = kv.first; }
        }
        if (best < 2) break;
        size_t at_best = 0;
        for (const auto& kv : counts) at_best += kv.second == best;
        g_tied_rounds += at_best > 1;
        const uint64_t sym = next++;
        const size_t before = t.size();
        const uint64_t rep = repair_apply_rule(t, bp.l, bp.r, sym);
        if (t.size() >= before || rep == 0) break;
        rules[4 * nr + 0] = sym; rules[4 * nr + 1] = bp.l; rules[4 * nr + 2] = bp.r; rules[4 * nr + 3] = best;
        nr++;
    }
    *out_len = t.size();
    *max_pair = maxf;
    if (seq_out) std::copy(t.begin(), t.end(), seq_out);
    return nr;
}

// apply_existing_grammar: every rule in order, greedy left to right.
uint64_t oc_repair_apply(const uint8_t* raw, uint64_t n, int storage_bytes, uint32_t masked_bits,
                         const uint64_t* rules, uint32_t n_rules, uint64_t* seq_out) {
    std::vector<uint64_t> t = repair_masked_words(raw, n, storage_bytes, masked_bits);
    for (uint32_t i = 0; i < n_rules; i++) repair_apply_rule(t, rules[4 * i + 1], rules[4 * i + 2], rules[4 * i]);
    if (seq_out) std::copy(t.begin(), t.end(), seq_out);
    return t.size();
}

}  // extern "C"
