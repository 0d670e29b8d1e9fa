// checkers_amd/csrc/ckr_api.cpp — the extern "C" layer (include/checkers_amd.h).
//
// Host responsibilities: argument checks, workspace carving, the histogram →
// table step (host code, as in the reference), and batching of encode units
// so the lane scratch stays within a fixed budget whatever the tensor size.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <map>
#include <mutex>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <functional>
#include <vector>

#include "checkers_amd.h"
#include "ckr_internal.h"
#include "ckr_table.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

}  // namespace

int ckr::set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

namespace {

#define CKR_HIP(call)                                                                      \
    do {                                                                                   \
        hipError_t _e = (call);                                                            \
        if (_e != hipSuccess)                                                              \
            return fail(CKR_E_HIP, "[ckr] HIP error in %s: %s", #call, hipGetErrorString(_e)); \
    } while (0)

constexpr uint64_t kAlign = 256;
constexpr uint64_t kScratchBudget = 2ull << 30;  // lane scratch per encode batch

inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned_to(const void* p, uint64_t a) { return a == 0 || reinterpret_cast<uintptr_t>(p) % a == 0; }

// Device-pointer check before anything is launched on a caller's buffer.  The
// reference validates each tensor pointer with hipPointerGetAttributes before
// its kernels run (src/ANSCompressor.cpp:567-585, :1177-1202), so that a
// freed or foreign pointer is an error instead of a GPU fault; here the byte
// range [p, p + bytes) must also lie inside the allocation holding p.  A
// failed query leaves an error in the runtime's last-error slot, which would
// be taken for a failed launch later, so it is cleared.
int check_buffer(const void* p, uint64_t bytes, const char* what) {
    if (bytes == 0) return CKR_OK;
    if (!p) return fail(CKR_E_INVALID, "[ckr] null %s pointer", what);
    // device memory: its allocation's range (one query); anything else (pinned
    // host memory, which the range query does not cover, or no allocation at
    // all): the pointer's type
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) == hipSuccess && base) {
        const uintptr_t b = reinterpret_cast<uintptr_t>(base), q = reinterpret_cast<uintptr_t>(p);
        if (q < b || q - b > size || bytes > size - (q - b))
            return fail(CKR_E_INVALID, "[ckr] %s [%p, +%llu bytes) runs past its allocation (%llu bytes at %p)", what, p,
                        (unsigned long long)bytes, (unsigned long long)size, base);
        return CKR_OK;
    }
    (void)hipGetLastError();
    hipPointerAttribute_t a;
    std::memset(&a, 0, sizeof(a));
    const hipError_t e = hipPointerGetAttributes(&a, p);
    if (e != hipSuccess || a.type == hipMemoryTypeUnregistered) {
        (void)hipGetLastError();
        return fail(CKR_E_INVALID, "[ckr] %s pointer %p is not device-accessible memory (%s)", what, p,
                    e != hipSuccess ? hipGetErrorString(e) : "unregistered host memory");
    }
    return CKR_OK;
}

// A source the kernels can read with 32-bit loads at its 4-byte columns.  A
// tensor that is only element-aligned (a 16-bit or 8-bit tensor starting at an
// address that is not a multiple of 4, e.g. a slice at an odd element offset
// of a flat buffer) is copied once into a stream-ordered aligned buffer, freed
// again in stream order after the last kernel that reads it.
struct Staged {
    const void* p = nullptr;
    void* tmp = nullptr;
    int make(const void* src, uint64_t bytes, hipStream_t s) {
        p = src;
        if (bytes == 0 || aligned_to(src, 4)) return CKR_OK;
        if (hipMallocAsync(&tmp, bytes, s) != hipSuccess) {
            (void)hipGetLastError();
            tmp = nullptr;
            return fail(CKR_E_HIP, "[ckr] staging buffer for an unaligned source (%llu bytes) unavailable",
                        (unsigned long long)bytes);
        }
        if (hipMemcpyAsync(tmp, src, bytes, hipMemcpyDeviceToDevice, s) != hipSuccess)
            return fail(CKR_E_HIP, "[ckr] staging copy of an unaligned source failed");
        p = tmp;
        return CKR_OK;
    }
    void release(hipStream_t s) {
        if (tmp) (void)hipFreeAsync(tmp, s);
        tmp = nullptr;
    }
};

bool dtype_ok(int dt) { return dt == CKR_F32 || dt == CKR_BF16 || dt == CKR_F16 || dt == CKR_I8 || dt == CKR_I32; }

// Unit geometry of a tensor; returns false (with the error set) for a unit size
// the format cannot express.
bool make_geom(uint64_t n_elems, int dtype, uint64_t unit_bytes, ckr::EncodeGeom* g) {
    const int es = ckr_element_size(dtype);
    g->es = es;
    g->spe = ckr_sidecar_bytes_per_elem(dtype);
    g->n_bytes = n_elems * (uint64_t)es;
    if (g->n_bytes == 0) { g->unit = 0; g->n_units = 0; g->wmax = 0; return true; }
    if (unit_bytes == 0 || unit_bytes >= g->n_bytes) {
        if (g->n_bytes > 0xFFFFFFFFull) {  // u32 byte_count / buf_offset (ANSCompressor.hpp:79-84)
            fail(CKR_E_INVALID, "[ckr] single-unit layout needs n_bytes < 2^32 (got %llu); use unit_bytes",
                 (unsigned long long)g->n_bytes);
            return false;
        }
        g->unit = g->n_bytes;
        g->n_units = 1;
    } else {
        if (unit_bytes % 256 != 0 || unit_bytes > 0xFFFFFFFFull) {
            fail(CKR_E_INVALID, "[ckr] unit_bytes must be a multiple of 256 below 2^32 (got %llu)",
                 (unsigned long long)unit_bytes);
            return false;
        }
        g->unit = unit_bytes;
        g->n_units = (g->n_bytes + unit_bytes - 1) / unit_bytes;
    }
    const uint64_t K = (g->unit + 255) / 256;  // symbols of lane 0
    g->wmax = (uint32_t)((2 * K + 3) / 4);     // worst case 2 bytes per symbol
    return true;
}

// Lane counts of the zero-plane canonical streams: full units (k0) and the two
// lane counts of the last unit (k1 = ceil, k2 = floor of its length / 256).
struct CanonKs {
    uint32_t k0, k1, k2, cw;
};
CanonKs canon_ks(const ckr::EncodeGeom& g) {
    CanonKs c{};
    if (g.n_units == 0) return c;
    const uint64_t last = g.n_bytes - (g.n_units - 1) * g.unit;
    c.k0 = (uint32_t)((g.unit + 255) / 256);
    c.k1 = (uint32_t)((last + 255) / 256);
    c.k2 = (uint32_t)(last / 256);
    c.cw = (2 * c.k0 + 3) / 4 + 1;
    return c;
}
constexpr uint32_t kDedupMaxK = 4096;  // zero-plane dedup up to 1 MiB units
constexpr uint32_t kFastMaxK = 256;    // LDS-staged encode / decode up to 64 KiB units
int g_fast_paths = 1;  // ckr_set_fast_paths: 0 general, 1 fast, 2 / 3 fast with minimal LDS slots (redo: general / fast)

bool use_dedup(const ckr::EncodeGeom& g) {
    return g_fast_paths && g.spe > 0 && g.n_units > 0 && (g.unit + 255) / 256 <= kDedupMaxK;
}
// Bytes of the canonical zero-plane stream of K symbols (the state update of
// rans_encode_kernel, ANSCompressor.cpp:180-202, for symbol 0, whose cum is 0).
uint32_t canon_stream_bytes(const ckr_freq_table* t, uint32_t K) {
    const uint32_t f = t->norm_freq[0];
    if (f == 0) return K;  // every symbol takes the raw-byte escape
    uint32_t x = CKR_L, bytes = 0;
    for (uint32_t k = 0; k < K; k++) {
        while (x >= (f << 19)) { bytes++; x >>= 8; }
        x = ((x / f) << CKR_SCALE_BITS) + (x % f);
    }
    return bytes;
}

// The canonical zero-plane entries (the layout canon_kernel writes: per lane
// count K, {K, final state, byte count, 0} and the stream in dword slots counted
// from its end, then the three streams in byte order) computed here from the
// reference's state update for symbol 0 (cum 0; f == 0: every symbol a raw
// byte).
void canon_host(const ckr_freq_table* t, const CanonKs& ck, std::vector<uint32_t>& out) {
    const uint32_t cw = ck.cw;
    out.assign(3 * (4 + cw) + 3 * cw, 0u);
    const uint32_t f = t->norm_freq[0];
    const uint32_t Ks[3] = {ck.k0, ck.k1, ck.k2};
    for (int e = 0; e < 3; e++) {
        uint32_t* base = out.data() + e * (4 + cw);
        uint32_t* slots = base + 4;
        uint32_t x = CKR_L, nacc = 0, w = 0;
        uint64_t acc = 0;
        auto push = [&](uint32_t byte) {
            acc = (acc << 8) | byte;
            if (++nacc == 4) { slots[w++] = (uint32_t)acc; nacc = 0; }
        };
        for (uint32_t k = 0; k < Ks[e]; k++) {
            if (f == 0) { push(0u); continue; }
            while (x >= (f << 19)) { push(x & 255u); x >>= 8; }
            x = ((x / f) << CKR_SCALE_BITS) + (x % f);
        }
        if (nacc) slots[w] = (uint32_t)acc;
        const uint32_t B = 4 * w + nacc, r = nacc;
        base[0] = Ks[e];
        base[1] = x;
        base[2] = B;
        base[3] = 0;
        uint32_t* sb = out.data() + 3 * (4 + cw) + e * cw;
        for (uint32_t d = 0; d < cw; d++) {
            uint32_t v = 0;
            for (uint32_t b = 0; b < 4; b++) {
                const uint32_t q = 4 * d + b;
                if (q >= B) break;
                const uint32_t slot = q < r ? w : w - 1 - ((q - r) >> 2);
                const uint32_t byte = q < r ? q : (q - r) & 3;
                v |= ((slots[slot] >> (8 * byte)) & 255u) << (8 * b);
            }
            sb[d] = v;
        }
    }
}

// Stores the host-computed entries with small kernels whose arguments carry
// them (CANON_ARG_DWORDS each: one launch for units up to 64 KiB).
hipError_t canon_launch(const ckr_freq_table* t, const CanonKs& ck, uint32_t* canon, hipStream_t s) {
    std::vector<uint32_t> w;
    canon_host(t, ck, w);
    ckr::CanonArg a;
    for (size_t off = 0; off < w.size(); off += ckr::CANON_ARG_DWORDS) {
        a.n = (uint32_t)std::min<size_t>(ckr::CANON_ARG_DWORDS, w.size() - off);
        a.off = (uint32_t)off;
        std::copy(w.begin() + off, w.begin() + off + a.n, a.w);
        const hipError_t e = ckr::launch_canon_store(a, canon, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

bool use_fast_encode(const ckr::EncodeGeom& g) { return use_dedup(g) && (g.unit + 255) / 256 <= kFastMaxK; }
// Units above 64 KiB (up to the dedup limit): the two-pass kernels.
bool use_seg_encode(const ckr::EncodeGeom& g) { return use_dedup(g) && (g.unit + 255) / 256 > kFastMaxK; }
// Units above the dedup limit (the one-stream layout of a tensor above 1 MiB):
// one chain per lane, then the segments side by side.
bool use_long_units(const ckr::EncodeGeom& g) {
    return g_fast_paths && g.spe > 0 && g.n_units > 0 && (g.unit + 255) / 256 > kDedupMaxK;
}

// A small pinned host buffer per thread and device for the few words the host
// reads back (histograms, control words, totals): copies into pinned memory are
// plain DMA, where pageable ones are staged by the runtime (~27 us each).
// Kept for the thread's life.
struct PinnedWords {
    uint32_t* w = nullptr;  // kPinnedWords words
};
constexpr uint32_t kPinnedWords = 2048;
// ckr_compress_many counts every histogram before any encode when no job is
// larger than this (cfg2's largest tensor, gate_proj, is 117 MB).
constexpr uint64_t kManySmallJobBytes = 256ull << 20;
uint32_t* pinned_words() {
    thread_local std::vector<PinnedWords> per_dev;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    if ((int)per_dev.size() <= dev) per_dev.resize(dev + 1);
    PinnedWords& p = per_dev[dev];
    if (!p.w && hipHostMalloc(reinterpret_cast<void**>(&p.w), kPinnedWords * 4, hipHostMallocDefault) != hipSuccess)
        p.w = nullptr;
    return p.w;
}

int max_lds_per_block() {
    static int v = -1;
    if (v < 0) {
        int dev = 0, x = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&x, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            x = 64 * 1024;
        v = x;
    }
    return v;
}

// LDS bytes reserved per live lane: the expected coded size of K symbols under
// the table plus six standard deviations (from the plane's histogram), or, with
// no histogram, K times the dearest symbol's cost.  A lane that still overflows
// only sends its unit through the general kernels.
uint32_t lane_slot_bytes(const uint32_t* plane_hist, const ckr_freq_table* t, uint32_t K) {
    double cost[256];
    for (int s = 0; s < 256; s++)
        cost[s] = t->norm_freq[s] ? std::log2((double)CKR_M / (double)t->norm_freq[s]) : 8.0;
    double bits;
    if (plane_hist) {
        double n = 0, m = 0, v = 0;
        for (int s = 0; s < 256; s++) { n += plane_hist[s]; m += plane_hist[s] * cost[s]; }
        if (n == 0) return 8;
        m /= n;
        for (int s = 0; s < 256; s++) v += plane_hist[s] * (cost[s] - m) * (cost[s] - m);
        v /= n;
        bits = K * m + 6.0 * std::sqrt(K * v) + 32.0;
    } else {
        double mx = 0;
        for (int s = 0; s < 256; s++) mx = std::max(mx, t->norm_freq[s] ? cost[s] : 0.0);
        bits = K * std::max(mx, 8.0) + 32.0;
    }
    uint64_t bytes = (uint64_t)std::ceil(bits / 8.0) + 8;
    bytes = (bytes + 3) & ~3ull;
    return (uint32_t)std::min<uint64_t>(std::max<uint64_t>(bytes, 8), 2ull * K + 8);
}

// Encode workspace: tables, histograms, canonical streams, the fast path's
// look-back state and redo list, and lane scratch for general-kernel batches
// (sized for the whole tensor's units, capped by kScratchBudget).
// The fast encoder's control words (ctl[0..5]) and, 8 words in, the device
// table's words (norm[256], sum, ambiguity, slot sizes), read back together.
constexpr uint32_t kCtlWords = 8 + ckr::kTinfoWords;
struct EncodeLayout {
    uint64_t off_enc, off_hist, off_canon, off_status, off_ctl, off_redo, off_usize, off_rec, off_aux, off_list,
        off_scratch, total;
    uint64_t batch_units;
};

EncodeLayout encode_layout(const ckr::EncodeGeom& g) {
    EncodeLayout L{};
    const uint64_t per_unit = (uint64_t)g.wmax * 256 * 4;
    uint64_t bu = per_unit ? std::max<uint64_t>(1, kScratchBudget / per_unit) : 1;
    bu = std::min<uint64_t>(bu, std::max<uint64_t>(g.n_units, 1));
    L.batch_units = bu;
    const CanonKs ck = canon_ks(g);
    uint64_t o = 0;
    L.off_enc = o;     o = align_up(o + 256 * sizeof(ckr::EncSym), kAlign);
    L.off_hist = o;    o = align_up(o + ckr::kHistTableWords * 4, kAlign);
    L.off_canon = o;   o = align_up(o + 3ull * (4 + 2 * ck.cw) * 4, kAlign);
    L.off_status = o;  o = align_up(o + ckr::encode_fast_status_words(g.n_units) * 8, kAlign);
    L.off_ctl = o;     o = align_up(o + kCtlWords * 4, kAlign);  // control words, then a device table's words
    L.off_redo = o;    o = align_up(o + g.n_units * 4, kAlign);
    const bool seg = use_seg_encode(g);  // two passes: checkpoint records instead of lane scratch
    const bool lng = use_long_units(g);  // likewise, one chain per lane
    L.off_usize = o;   o = align_up(o + (seg || lng ? g.n_units : bu) * 4, kAlign);
    L.off_rec = o;
    o = align_up(o + (seg ? g.n_units * ckr::encode_seg_segments(g.unit) * 128 * 8
                          : (lng ? ckr::encode_long_rec_bytes(g.n_units, g.unit) : 0)), kAlign);
    L.off_aux = o;     o = align_up(o + (seg || lng ? 512 : 0), kAlign);
    L.off_list = o;    o = align_up(o + (seg ? ckr::encode_seg_list_items(g.n_units, g.unit) * 8 : 0), kAlign);
    L.off_scratch = o; o = align_up(o + (seg || lng ? 0 : bu * per_unit), kAlign);
    L.total = o;
    return L;
}

// Decode workspace: enc table, canonical streams, decode table, bad-lane counter.
struct DecodeLayout {
    uint64_t off_canon, off_dec, off_bad, total;
    bool fast;
};
DecodeLayout decode_layout(const ckr::EncodeGeom& g) {
    DecodeLayout L{};
    const CanonKs ck = canon_ks(g);
    L.fast = g_fast_paths != 0 && g.spe > 0 && g.n_units > 0 && use_dedup(g);
    uint64_t o = 0;
    L.off_canon = o; o = align_up(o + (L.fast ? 3ull * (4 + 2 * ck.cw) * 4 : 0), kAlign);
    L.off_dec = o;   o = align_up(o + 4096 * 4, kAlign);
    L.off_bad = o;   o = align_up(o + 8, kAlign);
    L.total = o;
    return L;
}

bool table_arg(const ckr_freq_table* t, ckr::TableArg* a) {
    for (int s = 0; s < 256; s++) {
        if (t->norm_freq[s] > CKR_M) { fail(CKR_E_TABLE, "[ckr] norm_freq[%d]=%u > 4096", s, t->norm_freq[s]); return false; }
        a->norm[s] = (uint16_t)t->norm_freq[s];
    }
    for (int s = 0; s <= 256; s++) {
        if (t->cum_freq[s] > 0xFFFFu) { fail(CKR_E_TABLE, "[ckr] cum_freq[%d]=%u too large", s, t->cum_freq[s]); return false; }
        a->cum[s] = (uint16_t)t->cum_freq[s];
    }
    return true;
}

// ---- optional per-kernel timing
std::mutex g_prof_mu;
bool g_prof_on = false;
struct ProfRec {
    const char* name;
    hipEvent_t a, b;
};
std::vector<ProfRec> g_prof;
// phase stamps of fast-encode launches: {device buffer, units, stream}
struct PhaseRec {
    uint64_t* buf;
    uint64_t n;
    hipStream_t s;
};
std::vector<PhaseRec> g_phase;

}  // namespace

namespace ckr {
bool profiling() { return g_prof_on; }
// Set while a no-allocation entry point runs on this thread: profiling, which
// creates events and buffers, stays out of it.
thread_local bool t_noalloc = false;
void prof_mark(const char* name, hipStream_t s, bool begin) {
    if (!g_prof_on || t_noalloc) return;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return;
    (void)hipEventRecord(e, s);
    if (begin) g_prof.push_back({name, e, nullptr});
    else if (!g_prof.empty() && g_prof.back().b == nullptr) g_prof.back().b = e;
    else (void)hipEventDestroy(e);
}
uint64_t* prof_phase_buffer(uint64_t n, hipStream_t s) {
    // per-unit phase stamps are extra work inside the encoder, so they are taken
    // only on request (CKR_PROFILE_PHASES=1): the kernel times are then those of
    // the kernel as it runs without profiling
    static const bool phases = [] {
        const char* v = std::getenv("CKR_PROFILE_PHASES");
        return v && v[0] == '1';
    }();
    if (!g_prof_on || !phases || t_noalloc || n == 0) return nullptr;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    void* p = nullptr;
    if (hipMalloc(&p, n * 8) != hipSuccess) return nullptr;
    if (hipMemsetAsync(p, 0, n * 8, s) != hipSuccess) { (void)hipFree(p); return nullptr; }
    g_phase.push_back({static_cast<uint64_t*>(p), n / 8, s});
    return static_cast<uint64_t*>(p);
}
}  // namespace ckr

extern "C" {

int ckr_profile_begin(void) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    for (auto& r : g_prof) { (void)hipEventDestroy(r.a); if (r.b) (void)hipEventDestroy(r.b); }
    g_prof.clear();
    g_prof_on = true;
    return CKR_OK;
}

// Writes one line per kernel name: "<name> <launches> <total_ms>\n".
int ckr_profile_end(char* buf, uint64_t buflen) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof_on = false;
    std::map<std::string, std::pair<uint64_t, double>> agg;
    for (auto& r : g_prof) {
        if (r.b) {
            if (hipEventSynchronize(r.b) != hipSuccess) return fail(CKR_E_HIP, "[ckr] profile event sync failed");
            float ms = 0.f;
            (void)hipEventElapsedTime(&ms, r.a, r.b);
            auto& v = agg[r.name];
            v.first++;
            v.second += ms;
            (void)hipEventDestroy(r.b);
        }
        (void)hipEventDestroy(r.a);
    }
    g_prof.clear();
    // fast-encode phases: mean per unit (us) of the coders' wait for a free set,
    // coding, the hand-over to the packers, look-back, packing (thread 0), the
    // packers' closing barrier, and the chunks thread 0 packed
    {
        constexpr int NS = 8;
        double sum[6] = {0, 0, 0, 0, 0, 0}, life = 0, chunks = 0;
        uint64_t units = 0;
        std::vector<float> code_t, look_t;  // for percentiles
        for (auto& pr : g_phase) {
            std::vector<uint64_t> h(pr.n * NS);
            if (hipStreamSynchronize(pr.s) == hipSuccess &&
                hipMemcpy(h.data(), pr.buf, h.size() * 8, hipMemcpyDeviceToHost) == hipSuccess) {
                for (uint64_t u = 0; u < pr.n; u++) {
                    const uint64_t* t = &h[NS * u];
                    if (!t[6]) continue;  // unit not stamped
                    for (int k = 0; k < 6; k++) sum[k] += t[k + 1] >= t[k] ? (double)(t[k + 1] - t[k]) * 0.01 : 0.0;
                    code_t.push_back(t[2] >= t[1] ? (float)(t[2] - t[1]) * 0.01f : 0.f);
                    look_t.push_back(t[4] >= t[3] ? (float)(t[4] - t[3]) * 0.01f : 0.f);
                    life += (double)(t[6] - t[0]) * 0.01;
                    chunks += (double)t[7];
                    units++;
                }
            }
            (void)hipFree(pr.buf);
        }
        g_phase.clear();
        if (units) {
            const char* nm[6] = {"encode_fast.phase_setwait_us", "encode_fast.phase_code_us",
                                 "encode_fast.phase_handoff_us", "encode_fast.phase_lookback_us",
                                 "encode_fast.phase_pack_us", "encode_fast.phase_release_us"};
            for (int k = 0; k < 6; k++) agg[nm[k]] = {units, sum[k] / 1000.0};
            agg["encode_fast.unit_lifetime_us"] = {units, life / 1000.0};
            agg["encode_fast.thread0_chunks"] = {units, chunks / 1000.0};
            // percentiles (reported as a "total" over one launch so that avg = value)
            auto pct = [](std::vector<float>& v, double q) {
                const size_t k = std::min(v.size() - 1, (size_t)(q * (double)(v.size() - 1)));
                std::nth_element(v.begin(), v.begin() + k, v.end());
                return (double)v[k];
            };
            const double qs[3] = {0.1, 0.5, 0.9};
            const char* qn[3] = {"p10", "p50", "p90"};
            for (int i = 0; i < 3; i++) {
                agg[std::string("encode_fast.code_us_") + qn[i]] = {1, pct(code_t, qs[i]) / 1000.0};
                agg[std::string("encode_fast.lookback_us_") + qn[i]] = {1, pct(look_t, qs[i]) / 1000.0};
            }
        }
    }
    std::string out;
    for (auto& kv : agg) {
        char line[256];
        std::snprintf(line, sizeof(line), "%s %llu %.6f\n", kv.first.c_str(), (unsigned long long)kv.second.first,
                      kv.second.second);
        out += line;
    }
    if (buf && buflen) {
        std::strncpy(buf, out.c_str(), buflen - 1);
        buf[buflen - 1] = 0;
    }
    return CKR_OK;
}

const char* ckr_last_error(void) { return g_last_error.c_str(); }

int ckr_set_fast_paths(int mode) {
    const int prev = g_fast_paths;
    g_fast_paths = (mode < 0 || mode > 3) ? 1 : mode;
    return prev;
}
const char* ckr_version(void) { return "checkers_amd 0.1 gfx950"; }

int ckr_element_size(int dtype) {
    switch (dtype) {
        case CKR_F32: return 4; case CKR_BF16: return 2; case CKR_F16: return 2;
        case CKR_I8: return 1; case CKR_I32: return 4; default: return 0;
    }
}

int ckr_sidecar_bytes_per_elem(int dtype) {
    switch (dtype) {
        case CKR_F32: return 2; case CKR_BF16: return 1; case CKR_F16: return 1; default: return 0;
    }
}

int ckr_extract_mantissa(const void* d_src, uint64_t n_elems, int dtype, void* d_masked, void* d_sidecar,
                         void* stream) {
    const int spe = ckr_sidecar_bytes_per_elem(dtype);
    if (!dtype_ok(dtype)) return fail(CKR_E_INVALID, "[ckr] unknown dtype %d", dtype);
    if (spe == 0) return fail(CKR_E_INVALID, "[ckr] dtype %d has no mantissa sidecar", dtype);
    if (n_elems == 0) return CKR_OK;
    if (!d_src || !d_masked || !d_sidecar) return fail(CKR_E_INVALID, "[ckr] null pointer");
    const int es = ckr_element_size(dtype);
    if (!aligned_to(d_src, es) || !aligned_to(d_masked, es))
        return fail(CKR_E_INVALID, "[ckr] source and masked copy must be aligned to the element size");
    int rc;
    if ((rc = check_buffer(d_src, n_elems * es, "source")) || (rc = check_buffer(d_masked, n_elems * es, "masked copy")) ||
        (rc = check_buffer(d_sidecar, n_elems * spe, "sidecar")))
        return rc;
    CKR_HIP(ckr::launch_extract_mantissa(static_cast<const uint8_t*>(d_src), n_elems, ckr_element_size(dtype), spe,
                                         static_cast<uint8_t*>(d_masked), static_cast<uint8_t*>(d_sidecar),
                                         (hipStream_t)stream));
    return CKR_OK;
}

int ckr_byte_histogram(const void* d_src, uint64_t n_elems, int dtype, uint32_t* d_hist, void* stream) {
    if (!dtype_ok(dtype)) return fail(CKR_E_INVALID, "[ckr] unknown dtype %d", dtype);
    if (!d_hist || (n_elems && !d_src)) return fail(CKR_E_INVALID, "[ckr] null pointer");
    const int es = ckr_element_size(dtype);
    if (!aligned_to(d_src, es) || !aligned_to(d_hist, 4))
        return fail(CKR_E_INVALID, "[ckr] source must be aligned to the element size, histogram to 4 bytes");
    int rc;
    if ((rc = check_buffer(d_src, n_elems * es, "source")) || (rc = check_buffer(d_hist, 1024, "histogram"))) return rc;
    CKR_HIP(ckr::launch_masked_hist(static_cast<const uint8_t*>(d_src), n_elems * (uint64_t)es, es,
                                    ckr_sidecar_bytes_per_elem(dtype), d_hist, nullptr, (hipStream_t)stream));
    return CKR_OK;
}

int ckr_byte_histogram_planes(const void* d_src, uint64_t n_elems, int dtype, uint32_t* d_hist, void* stream) {
    if (!dtype_ok(dtype)) return fail(CKR_E_INVALID, "[ckr] unknown dtype %d", dtype);
    if (!d_hist || (n_elems && !d_src)) return fail(CKR_E_INVALID, "[ckr] null pointer");
    const int es = ckr_element_size(dtype);
    if (!aligned_to(d_src, es) || !aligned_to(d_hist, 4))
        return fail(CKR_E_INVALID, "[ckr] source must be aligned to the element size, histogram to 4 bytes");
    int rc;
    if ((rc = check_buffer(d_src, n_elems * es, "source")) || (rc = check_buffer(d_hist, 768 * 4, "histogram")))
        return rc;
    const int spe = ckr_sidecar_bytes_per_elem(dtype);
    CKR_HIP(ckr::launch_masked_hist(static_cast<const uint8_t*>(d_src), n_elems * (uint64_t)es, es, spe, d_hist,
                                    spe ? d_hist + 256 : nullptr, (hipStream_t)stream));
    return CKR_OK;
}

int ckr_byte_histogram_raw(const void* d_bytes, uint64_t n_bytes, uint32_t* d_hist, void* stream) {
    return ckr_byte_histogram(d_bytes, n_bytes, CKR_I8, d_hist, stream);
}

}  // extern "C"

namespace {
// The rest of a table from its slot counts: cumulative counts, x_max and the
// decode slots (normalize_histogram's tail and build_tables,
// src/ANSCompressor.cpp:495-503).
void fill_table(const uint32_t* norm, ckr_freq_table* t) {
    t->cum_freq[0] = 0;
    for (int i = 0; i < 256; i++) { t->norm_freq[i] = norm[i]; t->cum_freq[i + 1] = t->cum_freq[i] + norm[i]; }
    for (int s = 0; s < 256; s++) {
        if (!norm[s]) continue;
        t->x_max[s] = CKR_NORM_BASE * norm[s];
        for (uint32_t j = t->cum_freq[s]; j < t->cum_freq[s + 1] && j < CKR_M; j++) {
            t->decode_sym[j] = (uint8_t)s;
            t->decode_freq[j] = norm[s];
            t->decode_cum[j] = t->cum_freq[s];
        }
    }
}

// The slot counts by ranks (ckr_table.h), one symbol at a time, as the device
// computes them one symbol per thread; true when a correction boundary cuts a
// group of equal fractional parts (then only libstdc++'s sort decides).
bool ranked_norm(const uint32_t* h, bool ensure_full, uint32_t* norm) {
    uint64_t total = 0;
    int distinct = 0;
    for (int i = 0; i < 256; i++) { total += h[i]; distinct += h[i] > 0; }
    for (int i = 0; i < 256; i++) norm[i] = 0;
    if ((ensure_full ? 256 : distinct) == 0) {
        norm[0] = CKR_M;
        return false;
    }
    ckr::NormStart r[256];
    double up[256], down[256];
    uint32_t assigned = 0;
    for (int i = 0; i < 256; i++) {
        r[i] = ckr::norm_start(h[i], total, ensure_full);
        up[i] = ckr::norm_key_up(r[i]);
        down[i] = ckr::norm_key_down(r[i]);
        assigned += r[i].norm;
    }
    bool amb = false;
    for (uint32_t i = 0; i < 256; i++) {
        const int f = ckr::norm_fix(r[i].norm, r[i].frac, r[i].inc, up, down, assigned);
        amb |= f == ckr::kNormAmbiguous;
        norm[i] = r[i].norm + (f == 1 ? 1u : 0u) - (f == -1 ? 1u : 0u);
    }
    return amb;
}
}  // namespace

extern "C" {

// ANSCompressor::normalize_histogram (src/ANSCompressor.cpp:416-503): proportional
// slots, then one correction pass ordered by libstdc++ std::sort of the
// fractional parts (descending, ties in the order that sort leaves them).
int ckr_build_table(const uint32_t* h, int ensure_full_alphabet, ckr_freq_table* t, uint32_t* h_table_sum) {
    if (!h || !t) return fail(CKR_E_INVALID, "[ckr] null pointer");
    std::memset(t, 0, sizeof(*t));
    uint64_t total = 0;
    int distinct = 0;
    for (int i = 0; i < 256; i++) { total += h[i]; distinct += h[i] > 0; }
    if ((ensure_full_alphabet ? 256 : distinct) == 0) {
        t->norm_freq[0] = CKR_M;
        for (int i = 1; i <= 256; i++) t->cum_freq[i] = CKR_M;
        t->x_max[0] = CKR_NORM_BASE * CKR_M;
        for (uint32_t j = 0; j < CKR_M; j++) { t->decode_sym[j] = 0; t->decode_freq[j] = CKR_M; t->decode_cum[j] = 0; }
        if (h_table_sum) *h_table_sum = CKR_M;
        return CKR_OK;
    }
    uint32_t norm[256] = {};
    uint32_t assigned = 0;
    for (int i = 0; i < 256; i++) {
        if (!ensure_full_alphabet && h[i] == 0) continue;
        uint32_t slots = total ? (uint32_t)((uint64_t)std::max(h[i], 1u) * CKR_M / total) : 0u;
        norm[i] = slots ? slots : 1u;
        assigned += norm[i];
    }
    struct Frac { int sym; double frac; };
    std::vector<Frac> fr;
    fr.reserve(256);
    for (int i = 0; i < 256; i++) {
        if (!norm[i]) continue;
        const double exact = total ? (double)std::max(h[i], 1u) * CKR_M / (double)total : 1.0;
        fr.push_back({i, exact - (double)(int)exact});
    }
    std::sort(fr.begin(), fr.end(), [](const Frac& a, const Frac& b) { return a.frac > b.frac; });
    if (assigned < CKR_M) {
        uint32_t rem = CKR_M - assigned;
        for (size_t k = 0; k < fr.size() && rem; k++, rem--) norm[fr[k].sym]++;
    } else if (assigned > CKR_M) {
        uint32_t rem = assigned - CKR_M;
        for (int k = (int)fr.size() - 1; k >= 0 && rem; k--)
            if (norm[fr[k].sym] > 1) { norm[fr[k].sym]--; rem--; }
    }
    fill_table(norm, t);
    if (h_table_sum) *h_table_sum = t->cum_freq[256];
    return CKR_OK;
}

int ckr_build_tables_device(const uint32_t* d_hists, uint64_t n, int ensure_full_alphabet, uint32_t* d_rows,
                            void* stream) {
    if (n == 0) return CKR_OK;
    if (!d_hists || !d_rows) return fail(CKR_E_INVALID, "[ckr] null pointer");
    if (!aligned_to(d_hists, 4) || !aligned_to(d_rows, 4)) return fail(CKR_E_INVALID, "[ckr] tables need 4-byte alignment");
    int rc;
    if ((rc = check_buffer(d_hists, n * 256 * 4, "histograms")) || (rc = check_buffer(d_rows, n * 258 * 4, "rows")))
        return rc;
    CKR_HIP(ckr::launch_tables(d_hists, n, ensure_full_alphabet, d_rows, (hipStream_t)stream));
    return CKR_OK;
}

int ckr_build_table_ranked(const uint32_t* h, int ensure_full_alphabet, ckr_freq_table* t, int* ambiguous) {
    if (!h || !t || !ambiguous) return fail(CKR_E_INVALID, "[ckr] null pointer");
    std::memset(t, 0, sizeof(*t));
    uint32_t norm[256];
    *ambiguous = ranked_norm(h, ensure_full_alphabet != 0, norm) ? 1 : 0;
    fill_table(norm, t);
    return CKR_OK;
}

uint64_t ckr_num_units(uint64_t n_elems, int dtype, uint64_t unit_bytes) {
    ckr::EncodeGeom g;
    if (!dtype_ok(dtype) || !make_geom(n_elems, dtype, unit_bytes, &g)) return 0;
    return g.n_units;
}

uint64_t ckr_encode_max_output_bytes(uint64_t n_elems, int dtype, uint64_t unit_bytes) {
    (void)unit_bytes;  // every unit is at most its own length (passthrough rule)
    return n_elems * (uint64_t)ckr_element_size(dtype);
}

uint64_t ckr_encode_workspace_bytes(uint64_t n_elems, int dtype, uint64_t unit_bytes) {
    ckr::EncodeGeom g;
    if (!dtype_ok(dtype) || !make_geom(n_elems, dtype, unit_bytes, &g)) return 0;
    return encode_layout(g).total;
}

}  // extern "C"

namespace {

// Encode with an optional pair of live-plane histograms (host) used to size the
// fast path's LDS slots.
// after_launch (may be null) runs once the encode kernels are queued, before
// the host waits for them: work for other streams goes in there.
using AfterLaunch = std::function<hipError_t()>;

// An encode whose read-backs are left queued (ckr_compress_many): the words the
// host checks go into pinned slots, read after one synchronisation for the
// whole batch by encode_complete, which also queues any redo batches.
struct EncodeDeferred {
    uint32_t* pin = nullptr;  // 8 words: [0..3] control words (fast) or [0] error flag (two-pass); [4..5] total
    int kind = 0;             // 0 none (empty tensor), 1 fast, 2 two-pass, 3 general
    const uint8_t* src = nullptr;
    ckr::EncodeGeom g{};
    const ckr::EncSym* enc = nullptr;
    const uint32_t* canon = nullptr;
    uint32_t cw = 0;
    uint32_t* scratch = nullptr;
    ckr_stream_header* hdrs = nullptr;
    uint32_t* usize = nullptr;
    uint64_t* unit_off = nullptr;
    uint8_t* out = nullptr;
    const uint32_t* redo = nullptr;
    uint64_t batch_units = 0;
    bool redo_fast = false;  // redo units go to the fast encoder with slots that hold any lane
    ckr::FastEncParamsHost fp{};
    uint64_t* status = nullptr;
    uint32_t* ctl = nullptr;
};
int encode_impl(const void* d_src, uint64_t n_elems, int dtype, const ckr_freq_table* h_table, uint64_t unit_bytes,
                uint8_t* d_out, uint64_t out_capacity, ckr_stream_header* d_headers, uint64_t* d_unit_offsets,
                uint8_t* d_sidecar, void* d_workspace, uint64_t workspace_bytes, uint64_t* h_total_out,
                const uint32_t* h_planes, void* stream, const AfterLaunch* after_launch = nullptr,
                EncodeDeferred* defer = nullptr, bool planes_size_only = false) {
    if (!dtype_ok(dtype)) return fail(CKR_E_INVALID, "[ckr] unknown dtype %d", dtype);
    ckr::EncodeGeom g;
    if (!make_geom(n_elems, dtype, unit_bytes, &g)) return CKR_E_INVALID;
    hipStream_t s = (hipStream_t)stream;
    if (!h_table || !d_unit_offsets) return fail(CKR_E_INVALID, "[ckr] null table or offsets");
    if (g.n_units == 0) {
        CKR_HIP(ckr::launch_set_u64(d_unit_offsets, 0, s));
        if (h_total_out) *h_total_out = 0;
        if (defer) {
            defer->kind = 0;
            std::memset(defer->pin, 0, 32);
        }
        return CKR_OK;
    }
    if (!d_src || !d_out || !d_headers || !d_workspace) return fail(CKR_E_INVALID, "[ckr] null pointer");
    if (!aligned_to(d_src, 4) || !aligned16(d_workspace) || (d_sidecar && !aligned16(d_sidecar)))
        return fail(CKR_E_INVALID, "[ckr] sidecar and workspace must be 16-byte aligned");
    if (out_capacity < g.n_bytes)
        return fail(CKR_E_CAPACITY, "[ckr] output capacity %llu < %llu", (unsigned long long)out_capacity,
                    (unsigned long long)g.n_bytes);
    const EncodeLayout L = encode_layout(g);
    if (workspace_bytes < L.total)
        return fail(CKR_E_CAPACITY, "[ckr] workspace %llu < %llu", (unsigned long long)workspace_bytes,
                    (unsigned long long)L.total);
    ckr::TableArg ta;
    if (!table_arg(h_table, &ta)) return CKR_E_TABLE;
    uint8_t* ws = static_cast<uint8_t*>(d_workspace);
    auto* enc = reinterpret_cast<ckr::EncSym*>(ws + L.off_enc);
    auto* canon = reinterpret_cast<uint32_t*>(ws + L.off_canon);
    auto* usize = reinterpret_cast<uint32_t*>(ws + L.off_usize);
    auto* scratch = reinterpret_cast<uint32_t*>(ws + L.off_scratch);
    const bool dedup = use_dedup(g);
    const CanonKs ck = canon_ks(g);
    uint8_t* side = g.spe ? d_sidecar : nullptr;
    // escapes are possible unless the data's own live-plane histograms show
    // every symbol it contains has a slot
    // (planes_size_only: the histograms are a caller's, used for slot sizes only)
    bool escapes = true;
    if (h_planes && !planes_size_only) {
        escapes = false;
        for (int s2 = 0; s2 < 256; s2++)
            if ((h_planes[s2] || h_planes[256 + s2]) && !h_table->norm_freq[s2]) escapes = true;
    }
    bool fast = use_fast_encode(g);
    ckr::FastEncParamsHost fp{};
    if (fast) {
        fp.escapes = escapes;
        const uint32_t K = (uint32_t)((g.unit + 255) / 256);
        fp.cw = ck.cw;
        const uint32_t cbmax = std::max(canon_stream_bytes(h_table, ck.k0),
                                        std::max(canon_stream_bytes(h_table, ck.k1), canon_stream_bytes(h_table, ck.k2)));
        fp.canon_bytes = std::min<uint32_t>((cbmax + 3) & ~3u, 4 * ck.cw);
        if (g_fast_paths >= 2) {
            fp.sl0 = fp.sl1 = 8;
        } else {
            fp.sl0 = lane_slot_bytes(h_planes, h_table, K);
            fp.sl1 = lane_slot_bytes(h_planes ? h_planes + 256 : nullptr, h_table, K);
        }
        fast = ckr::encode_fast_lds_bytes(fp, (uint32_t)max_lds_per_block()) != 0;
    }
    // the fast encoder's look-back status and control words are cleared by the
    // launch that builds the encode entries
    if (fast)
        CKR_HIP(ckr::launch_build_enc_table_reset(ta, enc, reinterpret_cast<uint64_t*>(ws + L.off_status), g.n_units,
                                                  reinterpret_cast<uint32_t*>(ws + L.off_ctl), s));
    else
        CKR_HIP(ckr::launch_build_enc_table(ta, enc, s));
    if (dedup) CKR_HIP(canon_launch(h_table, ck, canon, s));

    if (use_long_units(g)) {
        auto* aux = reinterpret_cast<uint32_t*>(ws + L.off_aux);
        CKR_HIP(ckr::launch_encode_long(static_cast<const uint8_t*>(d_src), g, enc, escapes,
                                        reinterpret_cast<uint2*>(ws + L.off_rec), d_headers, usize, d_unit_offsets,
                                        side, d_out, aux, s));
        if (after_launch) CKR_HIP((*after_launch)());
        if (defer) {  // completed as the two-pass encode is: error word, then the total
            defer->kind = 2;
            CKR_HIP(hipMemcpyAsync(defer->pin, aux, 4, hipMemcpyDeviceToHost, s));
            CKR_HIP(hipMemcpyAsync(defer->pin + 4, d_unit_offsets + g.n_units, 8, hipMemcpyDeviceToHost, s));
            return CKR_OK;
        }
        uint32_t* pw = pinned_words();
        if (!pw) return fail(CKR_E_HIP, "[ckr] pinned host buffer unavailable");
        CKR_HIP(hipMemcpyAsync(pw, aux, 4, hipMemcpyDeviceToHost, s));
        CKR_HIP(hipMemcpyAsync(pw + 2, d_unit_offsets + g.n_units, 8, hipMemcpyDeviceToHost, s));
        CKR_HIP(hipStreamSynchronize(s));
        if (pw[0]) return fail(CKR_E_HIP, "[ckr] two-pass encode: a segment did not end at its checkpoint");
        if (h_total_out) std::memcpy(h_total_out, pw + 2, 8);
        return CKR_OK;
    }
    if (use_seg_encode(g)) {
        auto* rec = reinterpret_cast<uint2*>(ws + L.off_rec);
        auto* aux = reinterpret_cast<uint32_t*>(ws + L.off_aux);
        // Pass 2 of whole units on the fast encoder's waves: slots for 256 rows.
        // Pass 1 knows every lane's piece length, so a segment that does not fit
        // its slots simply goes to seg_code_kernel: the slots are made as large
        // as two coder pairs' LDS allows, starting from the plane histograms'
        // estimate and growing both planes alike.  Without plane histograms (a
        // caller's table) the two planes' needs are unknown and an even split
        // sends most segments of high-entropy data to seg_code_kernel, so
        // seg_code_kernel takes all of pass 2.  Mode 2 keeps minimal slots, so
        // that every segment takes seg_code_kernel.
        ckr::FastEncParamsHost sp{};
        sp.escapes = escapes;
        sp.cw = ck.cw;
        // the whole units' zero-plane lanes share one canonical stream (k0 symbols)
        sp.canon_bytes = std::min<uint32_t>((canon_stream_bytes(h_table, ck.k0) + 3) & ~3u, 4 * ck.cw);
        const uint32_t lds_limit = (uint32_t)max_lds_per_block();
        auto fits = [&](uint32_t a, uint32_t b) {
            sp.sl0 = a;
            sp.sl1 = b;
            return ckr::encode_seg_fast_lds_bytes(sp, lds_limit) != 0;
        };
        uint32_t a = 8, b = 8;
        if (g_fast_paths < 2) {
            constexpr uint32_t cap = 2 * 256 + 8;  // the most 256 symbols can emit, and the final dword
            if (h_planes) {
                a = std::min(cap, lane_slot_bytes(h_planes, h_table, 256));
                b = std::min(cap, lane_slot_bytes(h_planes + 256, h_table, 256));
            }
            while (!fits(a, b) && (a > 8 || b > 8)) (a >= b ? a : b) -= 4;
            while ((a < cap || b < cap) && fits(std::min(a + 4, cap), std::min(b + 4, cap))) {
                a = std::min(a + 4, cap);
                b = std::min(b + 4, cap);
            }
        }
        const bool seg_fast = (h_planes || g_fast_paths >= 2) && fits(a, b);
        CKR_HIP(ckr::launch_encode_seg(static_cast<const uint8_t*>(d_src), g, enc, canon, ck.cw, escapes, rec,
                                       d_headers, usize, d_unit_offsets, side, d_out, aux, seg_fast ? &sp : nullptr,
                                       lds_limit, aux + 64, ws + L.off_list, s));
        if (after_launch) CKR_HIP((*after_launch)());
        if (defer) {
            defer->kind = 2;
            CKR_HIP(hipMemcpyAsync(defer->pin, aux, 4, hipMemcpyDeviceToHost, s));
            CKR_HIP(hipMemcpyAsync(defer->pin + 4, d_unit_offsets + g.n_units, 8, hipMemcpyDeviceToHost, s));
            return CKR_OK;
        }
        uint32_t* pw = pinned_words();
        if (!pw) return fail(CKR_E_HIP, "[ckr] pinned host buffer unavailable");
        CKR_HIP(hipMemcpyAsync(pw, aux, 4, hipMemcpyDeviceToHost, s));
        CKR_HIP(hipMemcpyAsync(pw + 2, d_unit_offsets + g.n_units, 8, hipMemcpyDeviceToHost, s));
        CKR_HIP(hipStreamSynchronize(s));
        if (pw[0]) return fail(CKR_E_HIP, "[ckr] two-pass encode: a segment did not end at its checkpoint");
        if (h_total_out) std::memcpy(h_total_out, pw + 2, 8);
        return CKR_OK;
    }

    if (fast) {
        auto* status = reinterpret_cast<uint64_t*>(ws + L.off_status);
        auto* ctl = reinterpret_cast<uint32_t*>(ws + L.off_ctl);
        auto* redo = reinterpret_cast<uint32_t*>(ws + L.off_redo);
        CKR_HIP(ckr::launch_encode_fast(static_cast<const uint8_t*>(d_src), g, enc, canon, fp,
                                        (uint32_t)max_lds_per_block(), d_headers, side, d_out, d_unit_offsets, status,
                                        ctl, redo, s));
        // units whose lanes outgrew their LDS slots (the control words say how
        // many): coded again by the fast encoder with slots that hold any lane,
        // or, in mode 2 or when those slots do not fit, by the general kernels
        const bool redo_fast = g_fast_paths != 2 && ckr::encode_fast_list_fits(fp, g, (uint32_t)max_lds_per_block());
        if (after_launch) CKR_HIP((*after_launch)());
        if (defer) {
            defer->kind = 1;
            defer->src = static_cast<const uint8_t*>(d_src);
            defer->g = g;
            defer->enc = enc;
            defer->canon = canon;
            defer->cw = ck.cw;
            defer->scratch = scratch;
            defer->hdrs = d_headers;
            defer->usize = usize;
            defer->unit_off = d_unit_offsets;
            defer->out = d_out;
            defer->redo = redo;
            defer->batch_units = L.batch_units;
            defer->redo_fast = redo_fast;
            defer->fp = fp;
            defer->status = status;
            defer->ctl = ctl;
            // the control words and, in ctl[4..5], the total: one read-back
            CKR_HIP(hipMemcpyAsync(defer->pin, ctl, 24, hipMemcpyDeviceToHost, s));
            return CKR_OK;
        }
        // control words and the total (ctl[4..5]) in one read-back (the fast
        // kernel publishes every unit's offset, redo units included)
        uint32_t* pw = pinned_words();
        if (!pw) return fail(CKR_E_HIP, "[ckr] pinned host buffer unavailable");
        CKR_HIP(hipMemcpyAsync(pw, ctl, 24, hipMemcpyDeviceToHost, s));
        CKR_HIP(hipStreamSynchronize(s));
        uint32_t hctl[4];
        std::memcpy(hctl, pw, 16);
        if (hctl[2]) return fail(CKR_E_HIP, "[ckr] fast encode did not complete (flags %u: 1 look-back, 2 redo slots)", hctl[2]);
        if (h_total_out) std::memcpy(h_total_out, pw + 4, 8);
        // the redo units, at the offsets the fast kernel published
        if (hctl[1] && redo_fast)
            CKR_HIP(ckr::launch_encode_fast_list(static_cast<const uint8_t*>(d_src), g, enc, canon, fp,
                                                 (uint32_t)max_lds_per_block(), d_headers, d_out, d_unit_offsets,
                                                 status, ctl, redo, s));
        for (uint64_t r0 = 0; !redo_fast && r0 < hctl[1]; r0 += L.batch_units) {
            const uint64_t nb = std::min<uint64_t>(L.batch_units, hctl[1] - r0);
            CKR_HIP(ckr::launch_encode_batch(static_cast<const uint8_t*>(d_src), g, r0, nb, enc, canon, ck.cw, true,
                                             scratch, d_headers, nullptr, usize, d_unit_offsets, d_out, redo, s));
        }
        if (h_total_out && hctl[1]) CKR_HIP(hipStreamSynchronize(s));  // the output complete, as on the other paths
        return CKR_OK;
    } else {
        for (uint64_t u0 = 0; u0 < g.n_units; u0 += L.batch_units) {
            const uint64_t nb = std::min<uint64_t>(L.batch_units, g.n_units - u0);
            CKR_HIP(ckr::launch_encode_batch(static_cast<const uint8_t*>(d_src), g, u0, nb, enc, canon, ck.cw, dedup,
                                             scratch, d_headers, side, usize, d_unit_offsets, d_out, nullptr, s));
        }
        if (after_launch) CKR_HIP((*after_launch)());
    }
    if (defer) {
        defer->kind = 3;
        CKR_HIP(hipMemcpyAsync(defer->pin + 4, d_unit_offsets + g.n_units, 8, hipMemcpyDeviceToHost, s));
        return CKR_OK;
    }
    if (h_total_out) {
        uint32_t* pw = pinned_words();
        if (!pw) return fail(CKR_E_HIP, "[ckr] pinned host buffer unavailable");
        CKR_HIP(hipMemcpyAsync(pw, d_unit_offsets + g.n_units, 8, hipMemcpyDeviceToHost, s));
        CKR_HIP(hipStreamSynchronize(s));
        std::memcpy(h_total_out, pw, 8);
    }
    return CKR_OK;
}

// Output buffers of the jobs of one batched call ([lo, hi) device ranges):
// jobs run concurrently on several streams, so no two outputs may overlap,
// within a job or across jobs (inputs may be shared).
struct Span {
    uintptr_t lo, hi;
    uint64_t job;
    const char* what;
};
int check_disjoint(std::vector<Span>& v) {
    std::sort(v.begin(), v.end(), [](const Span& a, const Span& b) { return a.lo < b.lo; });
    uintptr_t hi = 0;
    size_t at = 0;
    for (size_t i = 0; i < v.size(); i++) {
        if (i && v[i].lo < hi)
            return fail(CKR_E_INVALID, "[ckr] job %llu's %s overlaps job %llu's %s", (unsigned long long)v[i].job,
                        v[i].what, (unsigned long long)v[at].job, v[at].what);
        if (v[i].hi > hi) {
            hi = v[i].hi;
            at = i;
        }
    }
    return CKR_OK;
}
void add_span(std::vector<Span>& v, const void* p, uint64_t bytes, uint64_t job, const char* what) {
    if (p && bytes) v.push_back({(uintptr_t)p, (uintptr_t)p + bytes, job, what});
}

// The caller buffers of an encode, checked before anything is queued: the
// source element-aligned and inside its allocation, the outputs and the
// workspace inside theirs at the sizes the header documents.
// An encode's arguments are checked in two parts: what its histogram and
// table set-up touch (sizes and alignment, the source and the workspace), and
// the output buffers, which the device-table paths check while that set-up
// runs (it writes nothing but the workspace).
int check_encode_inputs(const void* src, const ckr::EncodeGeom& g, uint64_t out_capacity, const void* ws,
                        uint64_t ws_bytes) {
    if (!aligned_to(src, (uint64_t)g.es))
        return fail(CKR_E_INVALID, "[ckr] source %p is not aligned to its element size (%d bytes)", src, g.es);
    if (g.n_units && out_capacity < g.n_bytes)
        return fail(CKR_E_CAPACITY, "[ckr] output capacity %llu < %llu", (unsigned long long)out_capacity,
                    (unsigned long long)g.n_bytes);
    if (g.n_units && ws_bytes < encode_layout(g).total)
        return fail(CKR_E_CAPACITY, "[ckr] workspace %llu < %llu", (unsigned long long)ws_bytes,
                    (unsigned long long)encode_layout(g).total);
    if (g.n_units == 0) return CKR_OK;
    int rc;
    if ((rc = check_buffer(src, g.n_bytes, "source")) || (rc = check_buffer(ws, ws_bytes, "workspace"))) return rc;
    return CKR_OK;
}
int check_encode_outputs(const ckr::EncodeGeom& g, uint64_t n_elems, const void* out, uint64_t out_capacity,
                         const void* hdrs, const void* offs, const void* side) {
    int rc;
    if ((rc = check_buffer(offs, (g.n_units + 1) * 8, "unit offsets"))) return rc;
    if (g.n_units == 0) return CKR_OK;
    if ((rc = check_buffer(out, out_capacity, "output")) ||
        (rc = check_buffer(hdrs, g.n_units * 256 * sizeof(ckr_stream_header), "headers")))
        return rc;
    if (side && g.spe && (rc = check_buffer(side, n_elems * (uint64_t)g.spe, "sidecar"))) return rc;
    return CKR_OK;
}
int check_encode_args(const void* src, const ckr::EncodeGeom& g, uint64_t n_elems, const void* out,
                      uint64_t out_capacity, const void* hdrs, const void* offs, const void* side, const void* ws,
                      uint64_t ws_bytes) {
    int rc = check_encode_inputs(src, g, out_capacity, ws, ws_bytes);
    return rc ? rc : check_encode_outputs(g, n_elems, out, out_capacity, hdrs, offs, side);
}

// After the stream has passed a deferred encode: its checks, its total, and the
// redo batches of the fast path (queued; the caller synchronises once more).
int encode_complete(const EncodeDeferred& d, uint64_t* total, bool* queued_more, hipStream_t s) {
    if (d.kind == 2 && d.pin[0]) return fail(CKR_E_HIP, "[ckr] two-pass encode: a segment did not end at its checkpoint");
    if (d.kind == 1) {
        if (d.pin[2]) return fail(CKR_E_HIP, "[ckr] fast encode did not complete (flags %u: 1 look-back, 2 redo slots)", d.pin[2]);
        if (d.pin[1] && d.redo_fast) {
            CKR_HIP(ckr::launch_encode_fast_list(d.src, d.g, d.enc, d.canon, d.fp, (uint32_t)max_lds_per_block(), d.hdrs,
                                                 d.out, d.unit_off, d.status, d.ctl, const_cast<uint32_t*>(d.redo), s));
            *queued_more = true;
        }
        for (uint64_t r0 = 0; !d.redo_fast && r0 < d.pin[1]; r0 += d.batch_units) {
            const uint64_t nb = std::min<uint64_t>(d.batch_units, d.pin[1] - r0);
            CKR_HIP(ckr::launch_encode_batch(d.src, d.g, r0, nb, d.enc, d.canon, d.cw, true, d.scratch, d.hdrs, nullptr,
                                             d.usize, d.unit_off, d.out, d.redo, s));
            *queued_more = true;
        }
    }
    std::memcpy(total, d.pin + 4, 8);
    return CKR_OK;
}

}  // namespace

extern "C" {

int ckr_encode(const void* d_src, uint64_t n_elems, int dtype, const ckr_freq_table* h_table, uint64_t unit_bytes,
               uint8_t* d_out, uint64_t out_capacity, ckr_stream_header* d_headers, uint64_t* d_unit_offsets,
               uint8_t* d_sidecar, void* d_workspace, uint64_t workspace_bytes, uint64_t* h_total_out,
               void* stream) {
    if (!dtype_ok(dtype)) return fail(CKR_E_INVALID, "[ckr] unknown dtype %d", dtype);
    ckr::EncodeGeom g;
    if (!make_geom(n_elems, dtype, unit_bytes, &g)) return CKR_E_INVALID;
    if (!h_table || !d_unit_offsets) return fail(CKR_E_INVALID, "[ckr] null table or offsets");
    int rc = check_encode_args(d_src, g, n_elems, d_out, out_capacity, d_headers, d_unit_offsets, d_sidecar, d_workspace,
                               workspace_bytes);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    Staged st;
    if ((rc = st.make(d_src, g.n_bytes, s))) return rc;
    rc = encode_impl(st.p, n_elems, dtype, h_table, unit_bytes, d_out, out_capacity, d_headers, d_unit_offsets,
                     d_sidecar, d_workspace, workspace_bytes, h_total_out, nullptr, stream);
    st.release(s);
    return rc;
}

}  // extern "C"

namespace {
int encode_planes_impl(const void* d_src, uint64_t n_elems, int dtype, const ckr_freq_table* h_table,
                       const uint32_t* h_planes, bool planes_cover_data, uint64_t unit_bytes, uint8_t* d_out,
                       uint64_t out_capacity, ckr_stream_header* d_headers, uint64_t* d_unit_offsets,
                       uint8_t* d_sidecar, void* d_workspace, uint64_t workspace_bytes, uint64_t* h_total_out,
                       void* stream) {
    if (!dtype_ok(dtype)) return fail(CKR_E_INVALID, "[ckr] unknown dtype %d", dtype);
    ckr::EncodeGeom g;
    if (!make_geom(n_elems, dtype, unit_bytes, &g)) return CKR_E_INVALID;
    if (!h_table || !d_unit_offsets) return fail(CKR_E_INVALID, "[ckr] null table or offsets");
    int rc = check_encode_args(d_src, g, n_elems, d_out, out_capacity, d_headers, d_unit_offsets, d_sidecar, d_workspace,
                               workspace_bytes);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    Staged st;
    if ((rc = st.make(d_src, g.n_bytes, s))) return rc;
    rc = encode_impl(st.p, n_elems, dtype, h_table, unit_bytes, d_out, out_capacity, d_headers, d_unit_offsets,
                     d_sidecar, d_workspace, workspace_bytes, h_total_out, g.spe ? h_planes : nullptr, stream,
                     nullptr, nullptr, !planes_cover_data);
    st.release(s);
    return rc;
}
}  // namespace

int ckr::encode_slice_of_counted(const void* d_src, uint64_t n_elems, int dtype, const ckr_freq_table* h_table,
                                 const uint32_t* h_planes, uint64_t unit_bytes, uint8_t* d_out, uint64_t out_capacity,
                                 ckr_stream_header* d_headers, uint64_t* d_unit_offsets, uint8_t* d_sidecar,
                                 void* d_workspace, uint64_t workspace_bytes, uint64_t* h_total_out, void* stream) {
    return encode_planes_impl(d_src, n_elems, dtype, h_table, h_planes, h_planes != nullptr, unit_bytes, d_out,
                              out_capacity, d_headers, d_unit_offsets, d_sidecar, d_workspace, workspace_bytes,
                              h_total_out, stream);
}

extern "C" {

int ckr_encode_planes(const void* d_src, uint64_t n_elems, int dtype, const ckr_freq_table* h_table,
                      const uint32_t* h_planes, uint64_t unit_bytes, uint8_t* d_out, uint64_t out_capacity,
                      ckr_stream_header* d_headers, uint64_t* d_unit_offsets, uint8_t* d_sidecar, void* d_workspace,
                      uint64_t workspace_bytes, uint64_t* h_total_out, void* stream) {
    return encode_planes_impl(d_src, n_elems, dtype, h_table, h_planes, false, unit_bytes, d_out, out_capacity,
                              d_headers, d_unit_offsets, d_sidecar, d_workspace, workspace_bytes, h_total_out, stream);
}

}  // extern "C"

namespace {
constexpr int kUseHostTable = 1;  // compress_device_table: take the host's sorted table instead

// The symbol-0 state chains of every count (ckr::launch_canon_chains), one
// buffer per device, made and filled on first use on the caller's stream (so
// that the first encode finds them filled) and kept for the process.
const void* canon_chains(hipStream_t s) {
    static std::mutex mu;
    static std::vector<void*> per_dev;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) { (void)hipGetLastError(); return nullptr; }
    std::lock_guard<std::mutex> lk(mu);
    if ((int)per_dev.size() <= dev) per_dev.resize(dev + 1, nullptr);
    if (!per_dev[dev]) {
        void* p = nullptr;
        if (hipMalloc(&p, ckr::kChainBytes) != hipSuccess) { (void)hipGetLastError(); return nullptr; }
        if (ckr::launch_canon_chains(p, s) != hipSuccess) { (void)hipGetLastError(); (void)hipFree(p); return nullptr; }
        per_dev[dev] = p;
    }
    return per_dev[dev];
}

// A tensor's encode with the table built on the device (tensors the fast
// encoder takes: masked dtypes, units of at most 64 KiB): from its histograms
// in device memory, the table by ranks, encode entries, canonical streams and
// slot sizes, and the encode are queued with no host round trip, and the
// control words and the table are read back into pinned words.  After the
// stream has passed them, dev_enc_finish takes the table and the total and
// queues any redo units; it returns kUseHostTable when the ranks leave the
// table to libstdc++'s sort (a correction boundary inside a group of equal
// fractional parts): the caller then encodes again under the host's sorted
// table, over the same outputs.
struct DevEnc {
    const uint8_t* src = nullptr;
    ckr::EncodeGeom g{};
    EncodeLayout L{};
    uint8_t* ws = nullptr;
    ckr::FastEncParamsHost fp{};
    CanonKs ck{};
    ckr_stream_header* hdrs = nullptr;
    uint64_t* unit_off = nullptr;
    uint8_t* out = nullptr;
    uint8_t* side = nullptr;
    uint32_t* dctl = nullptr;  // device: the control words, then the table's words (kCtlWords)
    uint32_t* pin = nullptr;   // their pinned host copy
    uint64_t epoch = 0;        // of the histogram and table launch (ctl[6..7] once the table is built)
    bool redo_queued = false;  // the list-mode redo pass follows the encode on its stream
};

// Whether the device table can serve this tensor, and its encode parameters
// (dctl: null for the workspace's own control words).
bool dev_enc_setup(DevEnc& d, const void* src, const ckr::EncodeGeom& g, uint8_t* ws, uint8_t* out,
                   ckr_stream_header* hdrs, uint64_t* unit_off, uint8_t* side, uint32_t* dctl, uint32_t* pin) {
    if (g_fast_paths != 1 || !use_fast_encode(g)) return false;
    d.src = static_cast<const uint8_t*>(src);
    d.g = g;
    d.L = encode_layout(g);
    d.ws = ws;
    d.ck = canon_ks(g);
    d.out = out; d.hdrs = hdrs; d.unit_off = unit_off; d.side = g.spe ? side : nullptr;
    d.dctl = dctl ? dctl : reinterpret_cast<uint32_t*>(ws + d.L.off_ctl);
    d.pin = pin;
    const uint32_t K = (uint32_t)((g.unit + 255) / 256);
    d.fp.escapes = false;  // the table is the data's own: every symbol present has a slot
    d.fp.cw = d.ck.cw;
    d.fp.canon_bytes = 4 * d.ck.cw;
    const uint32_t smax = ckr::encode_fast_max_slot(d.fp.canon_bytes, K, (uint32_t)max_lds_per_block());
    if (!smax || d.ck.cw > ckr::kCanonMaxCw) return false;
    d.fp.sl0 = d.fp.sl1 = smax;
    return ckr::encode_fast_lds_bytes(d.fp, (uint32_t)max_lds_per_block()) != 0;
}

// The table set-up of one tensor, for launch_hist_table.
ckr::TableEncJob dev_enc_table_job(const DevEnc& d, int ensure_full) {
    ckr::TableEncJob t{};
    t.enc = reinterpret_cast<ckr::EncSym*>(d.ws + d.L.off_enc);
    t.canon = reinterpret_cast<uint32_t*>(d.ws + d.L.off_canon);
    t.tinfo = d.dctl + 8;
    t.status = reinterpret_cast<uint64_t*>(d.ws + d.L.off_status);
    t.n_status = ckr::encode_fast_status_words(d.g.n_units);
    t.ctl = d.dctl;
    t.a = ckr::TableEncArg{(uint32_t)((d.g.unit + 255) / 256), d.ck.k0, d.ck.k1, d.ck.k2, d.ck.cw, d.fp.sl0, ensure_full};
    return t;
}

// The encode, after its table set-up on the same stream (or one that waited for it).
int dev_enc_queue_encode(const DevEnc& d, hipStream_t s) {
    const EncodeLayout& L = d.L;
    CKR_HIP(ckr::launch_encode_fast(d.src, d.g, reinterpret_cast<ckr::EncSym*>(d.ws + L.off_enc),
                                    reinterpret_cast<uint32_t*>(d.ws + L.off_canon), d.fp, (uint32_t)max_lds_per_block(),
                                    d.hdrs, d.side, d.out, d.unit_off, reinterpret_cast<uint64_t*>(d.ws + L.off_status),
                                    d.dctl, reinterpret_cast<uint32_t*>(d.ws + L.off_redo), s, d.dctl + 8 + 258));
    return CKR_OK;
}

// The encode and, right behind it with no read-back between them, the redo
// pass (it ends at once when no unit outgrew its slots).
int dev_enc_queue_encode_redo(DevEnc& d, hipStream_t s) {
    if (int rc = dev_enc_queue_encode(d, s)) return rc;
    const uint32_t lds_limit = (uint32_t)max_lds_per_block();
    if (ckr::encode_fast_list_fits(d.fp, d.g, lds_limit)) {
        const EncodeLayout& L = d.L;
        CKR_HIP(ckr::launch_encode_fast_list(d.src, d.g, reinterpret_cast<ckr::EncSym*>(d.ws + L.off_enc),
                                             reinterpret_cast<uint32_t*>(d.ws + L.off_canon), d.fp, lds_limit, d.hdrs,
                                             d.out, d.unit_off, reinterpret_cast<uint64_t*>(d.ws + L.off_status), d.dctl,
                                             reinterpret_cast<uint32_t*>(d.ws + L.off_redo), s));
        d.redo_queued = true;
    }
    return CKR_OK;
}

// The same encode as a job of launch_encode_fast_multi.
ckr::FastJob dev_fast_job(const DevEnc& d) {
    const EncodeLayout& L = d.L;
    ckr::FastJob f{};
    f.src = d.src;
    f.g = d.g;
    f.enc = reinterpret_cast<ckr::EncSym*>(d.ws + L.off_enc);
    f.canon = reinterpret_cast<uint32_t*>(d.ws + L.off_canon);
    f.hdrs = d.hdrs;
    f.sidecar = d.side;
    f.out = d.out;
    f.unit_off = d.unit_off;
    f.status = reinterpret_cast<uint64_t*>(d.ws + L.off_status);
    f.ctl = d.dctl;
    f.redo = reinterpret_cast<uint32_t*>(d.ws + L.off_redo);
    f.dsl = d.dctl + 8 + 258;
    f.sl0 = d.fp.sl0;
    f.sl1 = d.fp.sl1;
    f.cw = d.fp.cw;
    f.canon_bytes = d.fp.canon_bytes;
    return f;
}

int dev_enc_finish(const DevEnc& d, ckr_freq_table* h_table, uint64_t* h_total, bool* queued_more, hipStream_t s) {
    uint32_t hctl[8], ti[ckr::kTinfoWords];
    std::memcpy(hctl, d.pin, sizeof(hctl));
    std::memcpy(ti, d.pin + 8, sizeof(ti));
    if ((hctl[6] | (uint64_t)hctl[7] << 32) != d.epoch || (hctl[2] & 4u))
        return fail(CKR_E_HIP, "[ckr] histogram and table launch did not complete (flags %u)", hctl[2]);
    if (ti[257]) return kUseHostTable;
    if (hctl[2]) return fail(CKR_E_HIP, "[ckr] fast encode did not complete (flags %u: 1 look-back, 2 redo slots)", hctl[2]);
    if (h_table) {
        std::memset(h_table, 0, sizeof(*h_table));
        fill_table(ti, h_table);
    }
    if (h_total) std::memcpy(h_total, &hctl[4], 8);
    if (!hctl[1] || d.redo_queued) return CKR_OK;
    // units that outgrew their slots
    uint8_t* ws = d.ws;
    const EncodeLayout& L = d.L;
    auto* enc = reinterpret_cast<ckr::EncSym*>(ws + L.off_enc);
    auto* canon = reinterpret_cast<uint32_t*>(ws + L.off_canon);
    auto* status = reinterpret_cast<uint64_t*>(ws + L.off_status);
    auto* redo = reinterpret_cast<uint32_t*>(ws + L.off_redo);
    const uint32_t lds_limit = (uint32_t)max_lds_per_block();
    if (ckr::encode_fast_list_fits(d.fp, d.g, lds_limit)) {
        CKR_HIP(ckr::launch_encode_fast_list(d.src, d.g, enc, canon, d.fp, lds_limit, d.hdrs, d.out, d.unit_off, status,
                                             d.dctl, redo, s));
    } else {
        auto* usize = reinterpret_cast<uint32_t*>(ws + L.off_usize);
        auto* scratch = reinterpret_cast<uint32_t*>(ws + L.off_scratch);
        for (uint64_t r0 = 0; r0 < hctl[1]; r0 += L.batch_units) {
            const uint64_t nb = std::min<uint64_t>(L.batch_units, hctl[1] - r0);
            CKR_HIP(ckr::launch_encode_batch(d.src, d.g, r0, nb, enc, canon, d.ck.cw, true, scratch, d.hdrs, nullptr,
                                             usize, d.unit_off, d.out, redo, s));
        }
    }
    *queued_more = true;
    return CKR_OK;
}

// ckr_compress through the device table: histogram, queue, one synchronisation.
// check_outputs: the output buffers' checks, made while the histogram runs.
int compress_device_table(const void* src, const ckr::EncodeGeom& g, int ensure_full_alphabet, uint8_t* d_out,
                          ckr_stream_header* d_headers, uint64_t* d_unit_offsets, uint8_t* d_sidecar, uint8_t* ws,
                          ckr_freq_table* h_table, uint64_t* h_total_out, hipStream_t s,
                          const std::function<int()>& check_outputs) {
    uint32_t* pw = pinned_words();
    if (!pw) return fail(CKR_E_HIP, "[ckr] pinned host buffer unavailable");
    DevEnc d;
    if (!dev_enc_setup(d, src, g, ws, d_out, d_headers, d_unit_offsets, d_sidecar, nullptr, pw)) return kUseHostTable;
    const void* chains = canon_chains(s);
    if (!chains) return kUseHostTable;
    uint32_t* hist = reinterpret_cast<uint32_t*>(ws + d.L.off_hist);
    const ckr::HistSrc hs{d.src, g.n_bytes, g.es, (int)g.spe};
    const ckr::TableEncJob t = dev_enc_table_job(d, ensure_full_alphabet);
    CKR_HIP(ckr::launch_hist_table(&hs, &hist, &t, 1, chains, &d.epoch, s));
    int rc = check_outputs();
    if (rc) {
        (void)hipStreamSynchronize(s);  // the set-up writes the caller's workspace
        return rc;
    }
    rc = dev_enc_queue_encode_redo(d, s);
    if (rc) return rc;
    CKR_HIP(hipMemcpyAsync(pw, d.dctl, kCtlWords * 4, hipMemcpyDeviceToHost, s));
    CKR_HIP(hipStreamSynchronize(s));
    bool more = false;
    rc = dev_enc_finish(d, h_table, h_total_out, &more, s);
    if (rc == CKR_OK && more) CKR_HIP(hipStreamSynchronize(s));  // the output complete, as on the other paths
    return rc;
}
}  // namespace

extern "C" {

int ckr_compress(const void* d_src, uint64_t n_elems, int dtype, uint64_t unit_bytes, int ensure_full_alphabet,
                 uint8_t* d_out, uint64_t out_capacity, ckr_stream_header* d_headers, uint64_t* d_unit_offsets,
                 uint8_t* d_sidecar, void* d_workspace, uint64_t workspace_bytes, ckr_freq_table* h_table,
                 uint64_t* h_total_out, void* stream) {
    if (!dtype_ok(dtype)) return fail(CKR_E_INVALID, "[ckr] unknown dtype %d", dtype);
    ckr::EncodeGeom g;
    if (!make_geom(n_elems, dtype, unit_bytes, &g)) return CKR_E_INVALID;
    const EncodeLayout L = encode_layout(g);
    if (!d_workspace || workspace_bytes < L.total || !aligned16(d_workspace))
        return fail(CKR_E_CAPACITY, "[ckr] workspace too small or misaligned (%llu bytes, need %llu)",
                    (unsigned long long)workspace_bytes, (unsigned long long)L.total);
    if (n_elems && !d_src) return fail(CKR_E_INVALID, "[ckr] null source");
    if (!d_unit_offsets) return fail(CKR_E_INVALID, "[ckr] null offsets");
    int rc = check_encode_inputs(d_src, g, out_capacity, d_workspace, workspace_bytes);
    if (rc) return rc;
    const auto check_outputs = [&]() {
        return check_encode_outputs(g, n_elems, d_out, out_capacity, d_headers, d_unit_offsets, d_sidecar);
    };
    hipStream_t s = (hipStream_t)stream;
    Staged st;
    if ((rc = st.make(d_src, g.n_bytes, s))) return rc;
    // the fast encoder's tensors: the table on the device, no host round trip
    // before the encode (mode 1; modes 2 and 3 size the slots on the host)
    if (g_fast_paths == 1 && use_fast_encode(g)) {
        rc = compress_device_table(st.p, g, ensure_full_alphabet, d_out, d_headers, d_unit_offsets, d_sidecar,
                                   static_cast<uint8_t*>(d_workspace), h_table, h_total_out, s, check_outputs);
        if (rc != kUseHostTable) {
            st.release(s);
            return rc;
        }
    }
    if ((rc = check_outputs())) {
        st.release(s);
        return rc;
    }
    uint32_t* d_hist = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(d_workspace) + L.off_hist);
    const int es = ckr_element_size(dtype);
    hipError_t he = ckr::launch_masked_hist(static_cast<const uint8_t*>(st.p), n_elems * (uint64_t)es, es, g.spe, d_hist,
                                            d_hist + 256, s);
    uint32_t* pw = pinned_words();
    if (he == hipSuccess && pw) he = hipMemcpyAsync(pw, d_hist, 768 * 4, hipMemcpyDeviceToHost, s);
    if (he == hipSuccess && pw) he = hipStreamSynchronize(s);
    if (he != hipSuccess || !pw) {
        st.release(s);
        return pw ? fail(CKR_E_HIP, "[ckr] histogram failed: %s", hipGetErrorString(he))
                  : fail(CKR_E_HIP, "[ckr] pinned host buffer unavailable");
    }
    uint32_t hh[768];
    std::memcpy(hh, pw, sizeof(hh));
    ckr_freq_table local;
    ckr_freq_table* t = h_table ? h_table : &local;
    rc = ckr_build_table(hh, ensure_full_alphabet, t, nullptr);
    if (rc == CKR_OK)
        rc = encode_impl(st.p, n_elems, dtype, t, unit_bytes, d_out, out_capacity, d_headers, d_unit_offsets, d_sidecar,
                         d_workspace, workspace_bytes, h_total_out, g.spe ? hh + 256 : nullptr, stream);
    st.release(s);
    return rc;
}

// The second stream, its event and the pinned histogram buffers of
// ckr_compress_many, one set per device per thread (kept for the thread's life).
namespace {
struct ManyAux {
    hipStream_t s2 = nullptr;
    hipStream_t sx[2] = {nullptr, nullptr};  // with s2, the encodes of a shard of small tensors
    hipEvent_t ev = nullptr;
    hipEvent_t ev_prev = nullptr;  // the stream's work before the encode being queued
    hipEvent_t ev_tail = nullptr;  // a histogram's wider tail done (ckr_compress_many)
    uint32_t* pinned = nullptr;  // 2 x 768 words
    uint32_t* slots = nullptr;   // 8 words per job: the deferred read-backs
    uint64_t slot_jobs = 0;
    uint32_t* hists = nullptr;   // 768 words per job: histograms counted before any encode
    uint64_t hist_jobs = 0;
    uint32_t* d_hists = nullptr;  // their device copy (one grid counts them all)
    uint64_t d_hist_jobs = 0;
    uint32_t* tslots = nullptr;   // kCtlWords per job: device-table read-backs (pinned)
    uint32_t* d_tslots = nullptr; // their device side: every job's control and table words
    uint64_t tslot_jobs = 0;
    hipEvent_t ev_x[3] = {nullptr, nullptr, nullptr};  // s2, sx[0], sx[1] done (ckr_decode_many)
    uint64_t* bads = nullptr;    // ckr_decode_many's bad-lane counts, one per job
    uint64_t bad_jobs = 0;
    ckr::TableArg* dtabs = nullptr;    // ckr_decode_many's frequency tables, staged (pinned)
    ckr::TableArg* d_dtabs = nullptr;  // and on the device
    uint64_t dtab_jobs = 0;
    hipEvent_t ev_dtab = nullptr;      // their last upload done (the pinned copy may be reused)
};
hipError_t many_aux(ManyAux** out) {
    thread_local std::vector<ManyAux> per_dev;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if ((int)per_dev.size() <= dev) per_dev.resize(dev + 1);
    ManyAux& a = per_dev[dev];
    if (!a.s2) {
        if ((e = hipStreamCreateWithFlags(&a.s2, hipStreamNonBlocking)) != hipSuccess) return e;
        for (hipStream_t& x : a.sx)
            if ((e = hipStreamCreateWithFlags(&x, hipStreamNonBlocking)) != hipSuccess) return e;
        for (hipEvent_t& x : a.ev_x)
            if ((e = hipEventCreateWithFlags(&x, hipEventDisableTiming)) != hipSuccess) return e;
        if ((e = hipEventCreateWithFlags(&a.ev, hipEventDisableTiming)) != hipSuccess) return e;
        if ((e = hipEventCreateWithFlags(&a.ev_prev, hipEventDisableTiming)) != hipSuccess) return e;
        if ((e = hipEventCreateWithFlags(&a.ev_tail, hipEventDisableTiming)) != hipSuccess) return e;
        if ((e = hipEventCreateWithFlags(&a.ev_dtab, hipEventDisableTiming)) != hipSuccess) return e;
        if ((e = hipHostMalloc(reinterpret_cast<void**>(&a.pinned), 2 * 768 * sizeof(uint32_t), hipHostMallocDefault)) !=
            hipSuccess)
            return e;
    }
    *out = &a;
    return hipSuccess;
}
}  // namespace

static int set_job_error(int rc, uint64_t i) {
    return ckr::set_error(rc, "job " + std::to_string(i) + ": " + ckr_last_error());
}

int ckr_compress_many(ckr_compress_job* jobs, uint64_t n, uint64_t unit_bytes, int ensure_full_alphabet,
                      void* stream) {
    if (n == 0) return CKR_OK;
    if (!jobs) return fail(CKR_E_INVALID, "[ckr] null job list");
    if (n == 1) {  // one job: ckr_compress (which checks it) on the caller's stream, no second stream or events
        ckr_compress_job& jb = jobs[0];
        const int rc = ckr_compress(jb.d_src, jb.n_elems, jb.dtype, unit_bytes, ensure_full_alphabet, jb.d_out,
                                    jb.out_capacity, jb.d_headers, jb.d_unit_offsets, jb.d_sidecar, jb.d_workspace,
                                    jb.workspace_bytes, jb.h_table, &jb.total, stream);
        return rc ? set_job_error(rc, 0) : CKR_OK;
    }
    // every job's sizes, source and workspace checked before anything is
    // launched; its output buffers before anything writes them
    std::vector<ckr::EncodeGeom> geo(n);
    for (uint64_t i = 0; i < n; i++) {
        const ckr_compress_job& jb = jobs[i];
        if (!dtype_ok(jb.dtype)) return fail(CKR_E_INVALID, "[ckr] job %llu: unknown dtype %d", (unsigned long long)i, jb.dtype);
        if (!make_geom(jb.n_elems, jb.dtype, unit_bytes, &geo[i])) return CKR_E_INVALID;
        const EncodeLayout L = encode_layout(geo[i]);
        if (!jb.d_workspace || jb.workspace_bytes < L.total || !aligned16(jb.d_workspace))
            return fail(CKR_E_CAPACITY, "[ckr] job %llu: workspace too small or misaligned", (unsigned long long)i);
        if ((jb.n_elems && !jb.d_src) || !jb.d_unit_offsets)
            return fail(CKR_E_INVALID, "[ckr] job %llu: null source or offsets", (unsigned long long)i);
        const int rc = check_encode_inputs(jb.d_src, geo[i], jb.out_capacity, jb.d_workspace, jb.workspace_bytes);
        if (rc) return set_job_error(rc, i);
    }
    const auto check_outputs = [&]() -> int {
        for (uint64_t i = 0; i < n; i++) {
            const ckr_compress_job& jb = jobs[i];
            const int rc = check_encode_outputs(geo[i], jb.n_elems, jb.d_out, jb.out_capacity, jb.d_headers,
                                                jb.d_unit_offsets, jb.d_sidecar);
            if (rc) return set_job_error(rc, i);
        }
        return CKR_OK;
    };
    {  // jobs share no output or workspace bytes
        std::vector<Span> v;
        for (uint64_t i = 0; i < n; i++) {
            const ckr_compress_job& jb = jobs[i];
            const ckr::EncodeGeom& g = geo[i];
            add_span(v, jb.d_workspace, encode_layout(g).total, i, "workspace");
            add_span(v, jb.d_unit_offsets, (g.n_units + 1) * 8, i, "unit offsets");
            if (!g.n_units) continue;
            add_span(v, jb.d_out, g.n_bytes, i, "output");
            add_span(v, jb.d_headers, g.n_units * 256 * sizeof(ckr_stream_header), i, "headers");
            if (g.spe) add_span(v, jb.d_sidecar, jb.n_elems * (uint64_t)g.spe, i, "sidecar");
        }
        if (int rc = check_disjoint(v)) return rc;
    }
    hipStream_t s = (hipStream_t)stream;
    ManyAux* a = nullptr;
    CKR_HIP(many_aux(&a));
    // sources that are only element-aligned: aligned copies, queued before the
    // event the histogram stream waits for, freed once every job is complete
    std::vector<Staged> staged(n);
    struct Release {
        std::vector<Staged>& v;
        hipStream_t s, s2;
        ~Release() {
            bool any = false;
            for (auto& x : v) any = any || x.tmp;
            if (!any) return;
            (void)hipStreamSynchronize(s2);  // an error path may leave a histogram reading them
            for (auto& x : v) x.release(s);
        }
    } release_staged{staged, s, a->s2};
    // An error after the first launch leaves work queued on the library's
    // streams (encodes, histograms, read-backs into its pinned slots): every
    // stream is drained before the call returns, and before the staged copies
    // above are freed.
    struct Drain {
        ManyAux* a;
        hipStream_t s;
        bool ok = false;
        ~Drain() {
            if (ok) return;
            (void)hipStreamSynchronize(s);
            (void)hipStreamSynchronize(a->s2);
            for (hipStream_t x : a->sx) (void)hipStreamSynchronize(x);
        }
    } drain{a, s};
    for (uint64_t i = 0; i < n; i++) {
        const int rc = staged[i].make(jobs[i].d_src, geo[i].n_bytes, s);
        if (rc) return rc;
    }
    if (a->slot_jobs < n) {
        if (a->slots) CKR_HIP(hipHostFree(a->slots));
        a->slots = nullptr;
        a->slot_jobs = 0;
        CKR_HIP(hipHostMalloc(reinterpret_cast<void**>(&a->slots), n * 8 * sizeof(uint32_t), hipHostMallocDefault));
        a->slot_jobs = n;
    }
    std::vector<EncodeDeferred> defs(n);
    for (uint64_t i = 0; i < n; i++) defs[i].pin = a->slots + 8 * i;
    // the streams the encodes are queued on: the caller's, and in the
    // histograms-first mode below three of the library's as well
    std::vector<hipStream_t> enc_streams{s};
    // completes the encodes queued so far (jobs [0, upto)) once the streams have passed them
    auto complete = [&](uint64_t upto) -> int {
        for (hipStream_t x : enc_streams) CKR_HIP(hipStreamSynchronize(x));
        bool more = false;
        int first = CKR_OK;
        for (uint64_t k = 0; k < upto; k++) {
            const int r = encode_complete(defs[k], &jobs[k].total, &more, s);
            if (r && !first) first = r;
        }
        if (more) CKR_HIP(hipStreamSynchronize(s));
        return first;
    };
    CKR_HIP(hipEventRecord(a->ev, s));  // inputs ready in the caller's stream order
    CKR_HIP(hipStreamWaitEvent(a->s2, a->ev, 0));
    // job i's histogram words in its workspace (kHistTableWords; word 776 the
    // lean pass's chunk counter)
    auto hist_words = [&](uint64_t i) {
        return reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(jobs[i].d_workspace) + encode_layout(geo[i]).off_hist);
    };
    // tail: the lean pass in chunks that a tail (launch_masked_hist_join) can
    // join, the read-back left to the caller, behind that tail
    auto hist = [&](uint64_t i, uint32_t* h_dst, bool lean, bool tail) -> hipError_t {
        const ckr_compress_job& jb = jobs[i];
        uint32_t* d_hist = hist_words(i);
        const int es = ckr_element_size(jb.dtype);
        hipError_t e = ckr::launch_masked_hist(static_cast<const uint8_t*>(staged[i].p), jb.n_elems * (uint64_t)es, es,
                                               geo[i].spe, d_hist, d_hist + 256, a->s2, lean,
                                               tail ? d_hist + 776 : nullptr);
        if (e != hipSuccess || tail) return e;
        return hipMemcpyAsync(h_dst, d_hist, 768 * sizeof(uint32_t), hipMemcpyDeviceToHost, a->s2);
    };
    // Tables on the device when every job's tensor is one the fast encoder
    // takes (their control and table words in the library's pinned slots):
    // dev_setup sets chains (null: the host's tables serve the shard).
    std::vector<DevEnc> dv(n);
    const void* chains = nullptr;
    auto dev_setup = [&]() -> int {
        if (a->tslot_jobs < n) {
            if (a->tslots) CKR_HIP(hipHostFree(a->tslots));
            if (a->d_tslots) CKR_HIP(hipFree(a->d_tslots));
            a->tslots = nullptr;
            a->d_tslots = nullptr;
            a->tslot_jobs = 0;
            CKR_HIP(hipHostMalloc(reinterpret_cast<void**>(&a->tslots), n * kCtlWords * 4, hipHostMallocDefault));
            CKR_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_tslots), n * kCtlWords * 4));
            a->tslot_jobs = n;
        }
        bool all = true;
        for (uint64_t i = 0; i < n && all; i++)
            all = dev_enc_setup(dv[i], staged[i].p, geo[i], static_cast<uint8_t*>(jobs[i].d_workspace), jobs[i].d_out,
                                jobs[i].d_headers, jobs[i].d_unit_offsets, jobs[i].d_sidecar,
                                a->d_tslots + kCtlWords * i, a->tslots + kCtlWords * i);
        chains = all ? canon_chains(a->s2) : nullptr;
        return CKR_OK;
    };
    // Once every device-table encode is queued and the caller's stream waits
    // for them: one read-back of every job's words, then each job's table and
    // total; a job whose ranks leave its table to the sort is encoded again
    // under the host's table (hist_of(i): its 768 histogram words).
    auto dev_finish = [&](std::initializer_list<hipStream_t> streams,
                          const std::function<const uint32_t*(uint64_t)>& hist_of) -> int {
        CKR_HIP(hipMemcpyAsync(a->tslots, a->d_tslots, n * kCtlWords * 4, hipMemcpyDeviceToHost, s));
        for (hipStream_t x : streams) CKR_HIP(hipStreamSynchronize(x));
        bool more = false;
        for (uint64_t i = 0; i < n; i++) {
            ckr_compress_job& jb = jobs[i];
            int rc = dev_enc_finish(dv[i], jb.h_table, &jb.total, &more, s);
            if (rc == kUseHostTable) {  // the sorted table decides: encode this job again
                uint32_t hh[768];
                CKR_HIP(hipMemcpy(hh, hist_of(i), sizeof(hh), hipMemcpyDeviceToHost));
                ckr_freq_table local;
                ckr_freq_table* t = jb.h_table ? jb.h_table : &local;
                rc = ckr_build_table(hh, ensure_full_alphabet, t, nullptr);
                if (rc == CKR_OK)
                    rc = encode_impl(staged[i].p, jb.n_elems, jb.dtype, t, unit_bytes, jb.d_out, jb.out_capacity,
                                     jb.d_headers, jb.d_unit_offsets, jb.d_sidecar, jb.d_workspace, jb.workspace_bytes,
                                     &jb.total, hh + 256, s);
            }
            if (rc) return rc;
        }
        if (more) CKR_HIP(hipStreamSynchronize(s));
        drain.ok = true;
        return CKR_OK;
    };
    // A shard of small tensors: every histogram first (full width, back to
    // back), one synchronisation, then every encode queued without a host wait,
    // round robin over four streams.  Beside an encode of a few tens of
    // microseconds the host round trip from a histogram to the next table
    // (30-50 us) costs more than the histogram, and the encoder of a small
    // tensor has too few units to fill the device (a unit takes tens of
    // microseconds), so encodes of different tensors run side by side.  Each
    // job has its own workspace and outputs; the fast encoder's look-back waits
    // only for units whose tickets resident workgroups hold, so kernels that
    // share the device still finish.
    bool small = n > 1;
    for (uint64_t i = 0; i < n && small; i++) small = geo[i].n_bytes <= kManySmallJobBytes;
    if (small) {
        if (a->hist_jobs < n) {
            if (a->hists) CKR_HIP(hipHostFree(a->hists));
            a->hists = nullptr;
            a->hist_jobs = 0;
            CKR_HIP(hipHostMalloc(reinterpret_cast<void**>(&a->hists), n * 768 * sizeof(uint32_t), hipHostMallocDefault));
            a->hist_jobs = n;
        }
        if (a->d_hist_jobs < n) {  // no earlier call is still using it: each returns complete
            if (a->d_hists) CKR_HIP(hipFree(a->d_hists));
            a->d_hists = nullptr;
            a->d_hist_jobs = 0;
            CKR_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_hists), n * ckr::kHistTableWords * sizeof(uint32_t)));
            a->d_hist_jobs = n;
        }
        std::vector<ckr::HistSrc> hs(n);
        for (uint64_t i = 0; i < n; i++)
            hs[i] = {static_cast<const uint8_t*>(staged[i].p), geo[i].n_bytes, ckr_element_size(jobs[i].dtype),
                     (int)geo[i].spe};
        // tables on the device when every job's tensor is one the fast encoder
        // takes: no read-back or host table between the histograms and the
        // encodes
        if (int rc = dev_setup()) return rc;
        if (chains) {
            // every histogram and table in one grid (per 16 jobs), the tables
            // built by each job's last workgroup, then the encodes, then one
            // read-back of every job's control and table words
            std::vector<uint32_t*> hp(n);
            std::vector<ckr::TableEncJob> tj(n);
            std::vector<uint64_t> ep(n);
            for (uint64_t i = 0; i < n; i++) {
                hp[i] = a->d_hists + ckr::kHistTableWords * i;
                tj[i] = dev_enc_table_job(dv[i], ensure_full_alphabet);
            }
            CKR_HIP(ckr::launch_hist_table(hs.data(), hp.data(), tj.data(), (uint32_t)n, chains, ep.data(), a->s2));
            for (uint64_t i = 0; i < n; i++) dv[i].epoch = ep[i];
            if (int rc = check_outputs()) return rc;  // (the streams are drained on the way out)
            // the encodes of all jobs of one kind (spe, sidecar) in one launch
            // behind the tables, at most kMaxFastJobs a launch
            {
                std::vector<ckr::FastJob> fj[4];
                for (uint64_t i = 0; i < n; i++) {
                    if (!geo[i].n_units) continue;
                    const ckr::FastJob f = dev_fast_job(dv[i]);
                    fj[(f.g.spe == 2 ? 2 : 0) + (f.sidecar ? 1 : 0)].push_back(f);
                }
                for (auto& v : fj)
                    for (size_t o = 0; o < v.size(); o += ckr::kMaxFastJobs)
                        CKR_HIP(ckr::launch_encode_fast_multi(v.data() + o,
                                                              (uint32_t)std::min<size_t>(ckr::kMaxFastJobs, v.size() - o),
                                                              (uint32_t)max_lds_per_block(), a->s2));
            }
            CKR_HIP(hipEventRecord(a->ev, a->s2));  // the caller's stream waits for them
            CKR_HIP(hipStreamWaitEvent(s, a->ev, 0));
            return dev_finish({s, a->s2}, [&](uint64_t i) { return a->d_hists + ckr::kHistTableWords * i; });
        }
        if (int rc = check_outputs()) return rc;
        // every histogram in one grid (per 16 jobs) and one read-back: a launch
        // and a copy per job cost more host time than their kernels take
        CKR_HIP(ckr::launch_masked_hist_multi(hs.data(), (uint32_t)n, a->d_hists, a->s2));
        CKR_HIP(hipMemcpyAsync(a->hists, a->d_hists, n * 768 * sizeof(uint32_t), hipMemcpyDeviceToHost, a->s2));
        for (hipStream_t x : a->sx) CKR_HIP(hipStreamWaitEvent(x, a->ev, 0));  // inputs ready
        CKR_HIP(hipStreamSynchronize(a->s2));
        if (!g_prof_on) enc_streams = {s, a->s2, a->sx[0], a->sx[1]};
        for (uint64_t i = 0; i < n; i++) {
            ckr_compress_job& jb = jobs[i];
            const uint32_t* hh = a->hists + 768 * i;
            ckr_freq_table local;
            ckr_freq_table* t = jb.h_table ? jb.h_table : &local;
            int rc = ckr_build_table(hh, ensure_full_alphabet, t, nullptr);
            if (rc == CKR_OK)
                rc = encode_impl(staged[i].p, jb.n_elems, jb.dtype, t, unit_bytes, jb.d_out, jb.out_capacity,
                                 jb.d_headers, jb.d_unit_offsets, jb.d_sidecar, jb.d_workspace, jb.workspace_bytes,
                                 nullptr, geo[i].spe ? hh + 256 : nullptr, enc_streams[i % enc_streams.size()],
                                 nullptr, &defs[i]);
            if (rc) {
                (void)complete(i);
                return rc;
            }
        }
        drain.ok = true;  // complete() waits for every stream it queued on
        return complete(n);
    }
    if (int rc = check_outputs()) return rc;
    // Larger tensors: job i's encode goes on es[i % 2] (the caller's stream and
    // one of the library's), so that job i+1's encode takes the CUs that job
    // i's workgroups leave as its last units finish, instead of waiting for the
    // last of them.  Job i+1's histogram waits for job i-1's encode (the work
    // before job i's), so that it starts with job i's encode.  While
    // ckr_profile_begin is in effect every encode goes on the caller's stream
    // (here and in the small-shard mode above): a launch's profiling events
    // then bracket its own kernel and not the one still draining on another
    // stream.
    hipStream_t es[2] = {s, g_prof_on ? s : a->sx[0]};
    if (n > 1 && !g_prof_on) {
        CKR_HIP(hipStreamWaitEvent(a->sx[0], a->ev, 0));  // inputs ready
        enc_streams = {s, a->sx[0]};
    }
    CKR_HIP(hipEventRecord(a->ev_prev, s));  // before job 0's encode: the inputs
    CKR_HIP(hist(0, a->pinned, false, false));
    CKR_HIP(hipStreamSynchronize(a->s2));
    for (uint64_t i = 0; i < n; i++) {
        ckr_compress_job& jb = jobs[i];
        uint32_t* hh = a->pinned + 768 * (i & 1);
        ckr_freq_table local;
        ckr_freq_table* t = jb.h_table ? jb.h_table : &local;
        int rc = ckr_build_table(hh, ensure_full_alphabet, t, nullptr);
        if (rc) return rc;
        // job i + 1's histogram is queued once job i's encode kernels are, and
        // waits for job i-1's encode (the host does not wait for encodes), so
        // that it starts with job i's encode and the encoder's workgroups take
        // their CUs first
        bool queued = i + 1 >= n;
        // A histogram of more than 1.5 times the bytes of the encode it runs
        // beside outlasts it (the lean pass counts about as many bytes as
        // the encode reads, or a little more): once that encode is done it
        // gets three more workgroups per CU, on a third stream (nothing else
        // could use the device then, the next encode waiting for its table).
        // Queued at once, they would take CUs before the encode's workgroups
        // reach them.
        const bool tail = i + 1 < n && geo[i + 1].spe && 2 * geo[i + 1].n_bytes > 3 * geo[i].n_bytes;
        const AfterLaunch next = [&]() -> hipError_t {
            if (queued) return hipSuccess;
            queued = true;
            const hipError_t e2 = hipStreamWaitEvent(a->s2, a->ev_prev, 0);
            if (e2 != hipSuccess) return e2;
            return hist(i + 1, a->pinned + 768 * ((i + 1) & 1), true, tail);
        };
        // the encode is only queued: its read-backs are checked at the end, so
        // the next encode follows it on the stream without a host round trip
        rc = encode_impl(staged[i].p, jb.n_elems, jb.dtype, t, unit_bytes, jb.d_out, jb.out_capacity, jb.d_headers,
                         jb.d_unit_offsets, jb.d_sidecar, jb.d_workspace, jb.workspace_bytes, nullptr,
                         geo[i].spe ? hh + 256 : nullptr, es[i & 1], &next, &defs[i]);
        if (rc) {
            (void)hipStreamSynchronize(a->s2);
            (void)complete(i);
            return rc;
        }
        CKR_HIP(next());  // an empty job launches nothing
        CKR_HIP(hipEventRecord(a->ev_prev, es[i & 1]));  // job i queued: job i+2's histogram waits for it
        if (tail) {
            const ckr_compress_job& jn = jobs[i + 1];
            uint32_t* d_hist = hist_words(i + 1);
            const int esz = ckr_element_size(jn.dtype);
            CKR_HIP(hipStreamWaitEvent(a->sx[1], a->ev_prev, 0));
            CKR_HIP(ckr::launch_masked_hist_join(static_cast<const uint8_t*>(staged[i + 1].p),
                                                 jn.n_elems * (uint64_t)esz, esz, geo[i + 1].spe, d_hist, d_hist + 256,
                                                 d_hist + 776, 3, a->sx[1]));
            CKR_HIP(hipEventRecord(a->ev_tail, a->sx[1]));
            CKR_HIP(hipStreamWaitEvent(a->s2, a->ev_tail, 0));
            CKR_HIP(hipMemcpyAsync(a->pinned + 768 * ((i + 1) & 1), d_hist, 768 * sizeof(uint32_t),
                                   hipMemcpyDeviceToHost, a->s2));
        }
        if (i + 1 < n) CKR_HIP(hipStreamSynchronize(a->s2));
    }
    drain.ok = true;  // complete() waits for every stream it queued on
    return complete(n);
}

uint64_t ckr_decode_workspace_bytes(uint64_t n_elems, int dtype, uint64_t unit_bytes) {
    ckr::EncodeGeom g;
    if (!dtype_ok(dtype) || !make_geom(n_elems, dtype, unit_bytes, &g)) return 0;
    return decode_layout(g).total;
}

}  // extern "C"

namespace {
// ckr_decode and its no-allocation variant.  noalloc: the workspace is the
// device's scratch array, the destination must be 4-byte aligned (no staging
// copy), and the bad-lane count is read back through the caller's stack.
// A decode's arguments checked, with what its launches need (no launch).
struct DecPrep {
    ckr::EncodeGeom g{};
    DecodeLayout L{};
    ckr::TableArg ta{};
};
int decode_prepare(const uint8_t* d_data, const ckr_stream_header* d_headers, const uint64_t* d_unit_offsets,
                   const ckr_freq_table* h_table, uint64_t n_elems, int dtype, uint64_t unit_bytes,
                   const uint8_t* d_sidecar, void* d_dst, void* d_workspace, uint64_t workspace_bytes, DecPrep& p) {
    if (!dtype_ok(dtype)) return fail(CKR_E_INVALID, "[ckr] unknown dtype %d", dtype);
    ckr::EncodeGeom& g = p.g;
    if (!make_geom(n_elems, dtype, unit_bytes, &g)) return CKR_E_INVALID;
    if (g.n_units == 0) return CKR_OK;
    if (!h_table || !d_data || !d_headers || !d_unit_offsets || !d_dst || !d_workspace)
        return fail(CKR_E_INVALID, "[ckr] null pointer");
    if (g.spe && !d_sidecar) return fail(CKR_E_INVALID, "[ckr] dtype %d needs its sidecar", dtype);
    if (!aligned_to(d_dst, (uint64_t)g.es) || !aligned16(d_workspace) || (d_sidecar && !aligned16(d_sidecar)))
        return fail(CKR_E_INVALID, "[ckr] destination must be aligned to the element size, sidecar and workspace to 16 bytes");
    const DecodeLayout L = decode_layout(g);
    if (workspace_bytes < L.total) return fail(CKR_E_CAPACITY, "[ckr] decode workspace too small");
    if (h_table->cum_freq[256] != CKR_M)
        return fail(CKR_E_TABLE, "[ckr] table sums to %u, not 4096: stream not decodable", h_table->cum_freq[256]);
    {
        int rc;
        if ((rc = check_buffer(d_data, 1, "compressed data")) ||
            (rc = check_buffer(d_headers, g.n_units * 256 * sizeof(ckr_stream_header), "headers")) ||
            (rc = check_buffer(d_unit_offsets, (g.n_units + 1) * 8, "unit offsets")) ||
            (rc = check_buffer(d_dst, g.n_bytes, "destination")) || (rc = check_buffer(d_workspace, L.total, "workspace")))
            return rc;
        if (g.spe && (rc = check_buffer(d_sidecar, n_elems * (uint64_t)g.spe, "sidecar"))) return rc;
    }
    if (h_table->cum_freq[256] != CKR_M)
        return fail(CKR_E_TABLE, "[ckr] table sums to %u, not 4096: stream not decodable", h_table->cum_freq[256]);
    if (!table_arg(h_table, &p.ta)) return CKR_E_TABLE;
    p.L = L;
    return CKR_OK;
}

// counted: the caller reads the bad-lane count (h_bad_lanes, or
// ckr_decode_many's check), so that the fast decoder also compares the
// zero-plane lanes' bytes, which do not enter the output.
int decode_impl(const uint8_t* d_data, const ckr_stream_header* d_headers, const uint64_t* d_unit_offsets,
                const ckr_freq_table* h_table, uint64_t n_elems, int dtype, uint64_t unit_bytes,
                const uint8_t* d_sidecar, void* d_dst, void* d_workspace, uint64_t workspace_bytes,
                uint64_t* h_bad_lanes, void* stream, bool noalloc, bool counted) {
    if (h_bad_lanes) *h_bad_lanes = 0;
    DecPrep p;
    if (int rc = decode_prepare(d_data, d_headers, d_unit_offsets, h_table, n_elems, dtype, unit_bytes, d_sidecar, d_dst,
                                d_workspace, workspace_bytes, p))
        return rc;
    const ckr::EncodeGeom& g = p.g;
    if (g.n_units == 0) return CKR_OK;
    const DecodeLayout& L = p.L;
    const ckr::TableArg& ta = p.ta;
    hipStream_t s = (hipStream_t)stream;
    uint8_t* ws = static_cast<uint8_t*>(d_workspace);
    auto* canon = reinterpret_cast<uint32_t*>(ws + L.off_canon);
    auto* dec = reinterpret_cast<uint32_t*>(ws + L.off_dec);
    auto* bad = reinterpret_cast<unsigned long long*>(ws + L.off_bad);
    const CanonKs ck = canon_ks(g);
    CKR_HIP(ckr::launch_build_dec_table(ta, dec, bad, s));  // also clears the bad-lane counter
    if (L.fast) CKR_HIP(canon_launch(h_table, ck, canon, s));
    // the decoders store 32-bit words at the 4-byte columns of the destination:
    // a destination that is only element-aligned receives a copy
    uint8_t* out = static_cast<uint8_t*>(d_dst);
    void* tmp = nullptr;
    if (!aligned_to(d_dst, 4)) {
        if (noalloc) return fail(CKR_E_INVALID, "[ckr] the no-allocation decode needs a 4-byte aligned destination");
        if (hipMallocAsync(&tmp, g.n_bytes, s) != hipSuccess) {
            (void)hipGetLastError();
            return fail(CKR_E_HIP, "[ckr] staging buffer for an unaligned destination unavailable");
        }
        out = static_cast<uint8_t*>(tmp);
    }
    hipError_t de = use_long_units(g)
                        ? ckr::launch_decode_long(d_data, d_headers, d_unit_offsets, dec, g, d_sidecar, out, bad, s)
                        : ckr::launch_decode(d_data, d_headers, d_unit_offsets, dec, g, d_sidecar, out, bad,
                                             L.fast ? canon : nullptr, ck.cw, s, counted);
    if (tmp) {
        if (de == hipSuccess) de = hipMemcpyAsync(d_dst, tmp, g.n_bytes, hipMemcpyDeviceToDevice, s);
        (void)hipFreeAsync(tmp, s);
    }
    if (de != hipSuccess) return fail(CKR_E_HIP, "[ckr] decode launch failed: %s", hipGetErrorString(de));
    if (h_bad_lanes && noalloc) {
        unsigned long long nb = 0;
        CKR_HIP(hipMemcpyAsync(&nb, bad, 8, hipMemcpyDeviceToHost, s));
        CKR_HIP(hipStreamSynchronize(s));
        *h_bad_lanes = nb;
    } else if (h_bad_lanes) {
        uint32_t* pw = pinned_words();
        if (!pw) return fail(CKR_E_HIP, "[ckr] pinned host buffer unavailable");
        CKR_HIP(hipMemcpyAsync(pw, bad, 8, hipMemcpyDeviceToHost, s));
        CKR_HIP(hipStreamSynchronize(s));
        unsigned long long nb = 0;
        std::memcpy(&nb, pw, 8);
        *h_bad_lanes = nb;
    }
    return CKR_OK;
}

// The scratch of ckr_decode_noalloc: a file-scope device array, one copy per
// GPU the library runs on, held until the process ends.  Host code never
// passes `scratch` itself (on the host it is only a stand-in symbol): its
// device address is looked up once per device with hipGetSymbolAddress, with
// that device current, and that address is what the kernels receive.
constexpr uint64_t kNoAllocScratchBytes = 128 * 1024;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

int noalloc_scratch(void** out) {
    static std::mutex mu;
    static std::vector<void*> per_dev;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(CKR_E_HIP, "[ckr] no current device");
    std::lock_guard<std::mutex> lk(mu);
    if ((int)per_dev.size() <= dev) per_dev.resize(dev + 1, nullptr);
    if (!per_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return fail(CKR_E_HIP, "[ckr] scratch address lookup failed: %s", hipGetErrorString(e));
        }
        per_dev[dev] = p;
    }
    *out = per_dev[dev];
    return CKR_OK;
}
}  // namespace

extern "C" {

int ckr_decode(const uint8_t* d_data, const ckr_stream_header* d_headers, const uint64_t* d_unit_offsets,
               const ckr_freq_table* h_table, uint64_t n_elems, int dtype, uint64_t unit_bytes,
               const uint8_t* d_sidecar, void* d_dst, void* d_workspace, uint64_t workspace_bytes,
               uint64_t* h_bad_lanes, void* stream) {
    return decode_impl(d_data, d_headers, d_unit_offsets, h_table, n_elems, dtype, unit_bytes, d_sidecar, d_dst,
                       d_workspace, workspace_bytes, h_bad_lanes, stream, false, h_bad_lanes != nullptr);
}

int ckr_decode_many(ckr_decode_job* jobs, uint64_t n, uint64_t unit_bytes, int check, void* stream) {
    if (n == 0) return CKR_OK;
    if (!jobs) return fail(CKR_E_INVALID, "[ckr] null job list");
    for (uint64_t i = 0; i < n; i++) {
        ckr::EncodeGeom g;
        if (!dtype_ok(jobs[i].dtype) || !make_geom(jobs[i].n_elems, jobs[i].dtype, unit_bytes, &g))
            return fail(CKR_E_INVALID, "[ckr] job %llu: bad dtype or size", (unsigned long long)i);
        jobs[i].bad_lanes = 0;
    }
    {  // jobs share no destination or workspace bytes
        std::vector<Span> v;
        for (uint64_t i = 0; i < n; i++) {
            ckr::EncodeGeom g;
            make_geom(jobs[i].n_elems, jobs[i].dtype, unit_bytes, &g);
            if (!g.n_units) continue;
            add_span(v, jobs[i].d_workspace, decode_layout(g).total, i, "workspace");
            add_span(v, jobs[i].d_dst, g.n_bytes, i, "destination");
        }
        if (int rc = check_disjoint(v)) return rc;
    }
    hipStream_t s = (hipStream_t)stream;
    ManyAux* a = nullptr;
    CKR_HIP(many_aux(&a));
    // Jobs of up to 256 MiB each go round robin over four streams (the
    // caller's and three of the library's): a small tensor has too few units to
    // fill the device, and a unit takes tens of microseconds.  A larger job
    // fills the device by itself: then the jobs alternate between two streams,
    // so that job i+1 takes the CUs job i leaves as its last units finish
    // (cfg3 decode 6.42-6.47 -> 6.29 ms).  While ckr_profile_begin is in
    // effect every job goes on the caller's stream, so that a launch's
    // profiling events bracket its own kernel.
    bool small = true;
    for (uint64_t i = 0; i < n && small; i++) {
        ckr::EncodeGeom g;
        make_geom(jobs[i].n_elems, jobs[i].dtype, unit_bytes, &g);
        small = g.n_bytes <= kManySmallJobBytes;
    }
    std::vector<hipStream_t> pool{s};
    if (n > 1 && !g_prof_on) {
        if (small) pool = {s, a->s2, a->sx[0], a->sx[1]};
        else pool = {s, a->s2};
        CKR_HIP(hipEventRecord(a->ev, s));  // inputs ready in the caller's stream order
        for (size_t k = 1; k < pool.size(); k++) CKR_HIP(hipStreamWaitEvent(pool[k], a->ev, 0));
    }
    if (check && a->bad_jobs < n) {
        if (a->bads) CKR_HIP(hipHostFree(a->bads));
        a->bads = nullptr;
        a->bad_jobs = 0;
        CKR_HIP(hipHostMalloc(reinterpret_cast<void**>(&a->bads), n * sizeof(uint64_t), hipHostMallocDefault));
        a->bad_jobs = n;
    }
    // A shard of small tensors that the fast decoder takes whole (masked
    // dtypes of one kind or two, 4-byte aligned destinations; empty jobs have
    // nothing to decode): one set-up
    // launch for every job's decode table, canonical streams and bad-lane
    // counter, from the frequency tables uploaded in one copy, then one decode
    // launch over every job's units per dtype class, all on the caller's
    // stream.  The per-job launches otherwise came 10-20 us apart, slower than
    // the small decodes ran.  Any job that does not qualify, or fails its
    // checks, sends the shard the per-job way below.
    if (small && n > 1 && !g_prof_on) {
        std::vector<DecPrep> pp(n);
        bool all = true;
        for (uint64_t i = 0; i < n && all; i++) {
            const ckr_decode_job& jb = jobs[i];
            all = decode_prepare(jb.d_data, jb.d_headers, jb.d_unit_offsets, jb.h_table, jb.n_elems, jb.dtype,
                                 unit_bytes, jb.d_sidecar, jb.d_dst, jb.d_workspace, jb.workspace_bytes, pp[i]) == CKR_OK &&
                  (pp[i].g.n_units == 0 ||
                   (pp[i].L.fast && !use_long_units(pp[i].g) && aligned_to(jb.d_dst, 4)));
        }
        const void* chains = all ? canon_chains(s) : nullptr;
        if (all && chains) {
            if (a->dtab_jobs < n) {
                CKR_HIP(hipEventSynchronize(a->ev_dtab));
                if (a->dtabs) CKR_HIP(hipHostFree(a->dtabs));
                if (a->d_dtabs) CKR_HIP(hipFree(a->d_dtabs));
                a->dtabs = nullptr;
                a->d_dtabs = nullptr;
                a->dtab_jobs = 0;
                CKR_HIP(hipHostMalloc(reinterpret_cast<void**>(&a->dtabs), n * sizeof(ckr::TableArg), hipHostMallocDefault));
                CKR_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_dtabs), n * sizeof(ckr::TableArg)));
                a->dtab_jobs = n;
            }
            CKR_HIP(hipEventSynchronize(a->ev_dtab));  // the previous call's upload has left the pinned copy
            std::vector<ckr::DecSetupJob> sj;
            std::vector<uint64_t> sj_job;  // the job of each set-up
            std::vector<ckr::DecJob> dj[2];
            for (uint64_t i = 0; i < n; i++) {
                const ckr_decode_job& jb = jobs[i];
                const DecPrep& p = pp[i];
                if (!p.g.n_units) continue;
                const uint64_t k = sj.size();
                a->dtabs[k] = p.ta;
                uint8_t* ws = static_cast<uint8_t*>(jb.d_workspace);
                auto* canon = reinterpret_cast<uint32_t*>(ws + p.L.off_canon);
                auto* dec = reinterpret_cast<uint32_t*>(ws + p.L.off_dec);
                auto* bad = reinterpret_cast<unsigned long long*>(ws + p.L.off_bad);
                const CanonKs ck = canon_ks(p.g);
                sj.push_back(ckr::DecSetupJob{a->d_dtabs + k, dec, canon, bad, ck.k0, ck.k1, ck.k2, ck.cw});
                sj_job.push_back(i);
                ckr::DecJob d{};
                d.data = jb.d_data;
                d.hdrs = jb.d_headers;
                d.unit_off = jb.d_unit_offsets;
                d.dec = dec;
                d.canon = canon;
                d.sidecar = jb.d_sidecar;
                d.dst = static_cast<uint8_t*>(jb.d_dst);
                d.bad = bad;
                d.g = p.g;
                d.cw = ck.cw;
                d.zero_bytes = check ? 1u : 0u;
                dj[p.g.spe == 2 ? 1 : 0].push_back(d);
            }
            if (!sj.empty()) {
                CKR_HIP(hipMemcpyAsync(a->d_dtabs, a->dtabs, sj.size() * sizeof(ckr::TableArg), hipMemcpyHostToDevice, s));
                CKR_HIP(hipEventRecord(a->ev_dtab, s));
                CKR_HIP(ckr::launch_dec_setup_multi(sj.data(), (uint32_t)sj.size(), chains, s));
            }
            for (auto& v : dj)
                for (size_t o = 0; o < v.size(); o += ckr::kMaxDecJobs) {
                    const hipError_t e = ckr::launch_decode_fast_multi(
                        v.data() + o, (uint32_t)std::min<size_t>(ckr::kMaxDecJobs, v.size() - o), s);
                    if (e != hipSuccess) return fail(CKR_E_HIP, "[ckr] decode launch failed: %s", hipGetErrorString(e));
                }
            if (check) {
                for (size_t k = 0; k < sj.size(); k++)
                    CKR_HIP(hipMemcpyAsync(a->bads + k, sj[k].bad, 8, hipMemcpyDeviceToHost, s));
                CKR_HIP(hipStreamSynchronize(s));
                for (size_t k = 0; k < sj.size(); k++) jobs[sj_job[k]].bad_lanes = a->bads[k];
            }
            return CKR_OK;
        }
    }
    // every stream joins the caller's again, also when a job fails to queue
    auto join = [&]() -> hipError_t {
        for (size_t k = 1; k < pool.size(); k++) {
            hipError_t e = hipEventRecord(a->ev_x[k - 1], pool[k]);
            if (e == hipSuccess) e = hipStreamWaitEvent(s, a->ev_x[k - 1], 0);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    };
    for (uint64_t i = 0; i < n; i++) {
        const ckr_decode_job& jb = jobs[i];
        hipStream_t js = pool[i % pool.size()];
        int rc = decode_impl(jb.d_data, jb.d_headers, jb.d_unit_offsets, jb.h_table, jb.n_elems, jb.dtype, unit_bytes,
                             jb.d_sidecar, jb.d_dst, jb.d_workspace, jb.workspace_bytes, nullptr, js, false,
                             check != 0);
        if (rc == CKR_OK && check) {
            ckr::EncodeGeom g;
            make_geom(jb.n_elems, jb.dtype, unit_bytes, &g);
            a->bads[i] = 0;
            if (g.n_units) {
                const DecodeLayout L = decode_layout(g);
                if (hipMemcpyAsync(a->bads + i, static_cast<uint8_t*>(jb.d_workspace) + L.off_bad, 8,
                                   hipMemcpyDeviceToHost, js) != hipSuccess)
                    rc = fail(CKR_E_HIP, "[ckr] job %llu: bad-lane read-back failed", (unsigned long long)i);
            }
        }
        if (rc) {
            (void)join();
            return set_job_error(rc, i);
        }
    }
    CKR_HIP(join());
    if (check) {
        CKR_HIP(hipStreamSynchronize(s));
        for (uint64_t i = 0; i < n; i++) jobs[i].bad_lanes = a->bads[i];
    }
    return CKR_OK;
}

int ckr_decode_noalloc(const uint8_t* d_data, const ckr_stream_header* d_headers, const uint64_t* d_unit_offsets,
                       const ckr_freq_table* h_table, uint64_t n_elems, int dtype, uint64_t unit_bytes,
                       const uint8_t* d_sidecar, void* d_dst, uint64_t* h_bad_lanes, void* stream) {
    if (!dtype_ok(dtype)) return fail(CKR_E_INVALID, "[ckr] unknown dtype %d", dtype);
    ckr::EncodeGeom g;
    if (!make_geom(n_elems, dtype, unit_bytes, &g)) return CKR_E_INVALID;
    const uint64_t need = decode_layout(g).total;
    if (need > kNoAllocScratchBytes)
        return fail(CKR_E_CAPACITY, "[ckr] decode needs %llu bytes of scratch, above the no-allocation limit of %llu",
                    (unsigned long long)need, (unsigned long long)kNoAllocScratchBytes);
    if (g.n_units && d_dst && !aligned_to(d_dst, 4))
        return fail(CKR_E_INVALID, "[ckr] the no-allocation decode needs a 4-byte aligned destination");
    // the bad-lane count is read back with a synchronisation, which a stream
    // being captured into a graph cannot take: under capture it must be NULL
    if (h_bad_lanes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) {
            (void)hipGetLastError();
            return fail(CKR_E_HIP, "[ckr] cannot query the stream's capture status");
        }
        if (cs != hipStreamCaptureStatusNone)
            return fail(CKR_E_INVALID, "[ckr] h_bad_lanes must be NULL while the stream is captured (reading the "
                                       "count back needs a synchronisation)");
    }
    void* ws = nullptr;
    if (int rc = noalloc_scratch(&ws)) return rc;
    ckr::t_noalloc = true;
    const int rc = decode_impl(d_data, d_headers, d_unit_offsets, h_table, n_elems, dtype, unit_bytes, d_sidecar, d_dst,
                               ws, kNoAllocScratchBytes, h_bad_lanes, stream, true, h_bad_lanes != nullptr);
    ckr::t_noalloc = false;
    return rc;
}

// ---- analyzer: per record [p1 nblk][p2 nblk][params][hist partial nblk*256]
uint64_t ckr_analyze_workspace_bytes(const ckr_stats_record* recs, uint64_t n) {
    if (n && !recs) return 0;
    return ckr::analyze_workspace_bytes(recs, n);
}

int ckr_analyze(const ckr_stats_record* recs, uint64_t n, void* d_workspace, uint64_t workspace_bytes, void* stream) {
    if (n && !recs) return fail(CKR_E_INVALID, "[ckr] null records");
    const uint64_t need = ckr_analyze_workspace_bytes(recs, n);
    if (need && (!d_workspace || workspace_bytes < need)) return fail(CKR_E_CAPACITY, "[ckr] analyze workspace too small");
    for (uint64_t i = 0; i < n; i++) {
        const ckr_stats_record& r = recs[i];
        if (!r.d_ptr || !r.num_elements || !dtype_ok((int)r.data_type)) continue;  // skipped, as the reference does
        const int es = ckr_element_size((int)r.data_type);
        if (reinterpret_cast<uintptr_t>(r.d_ptr) % (uintptr_t)es)
            return fail(CKR_E_INVALID, "[ckr] record %llu: data pointer not aligned to its element size",
                        (unsigned long long)i);
    }
    CKR_HIP(ckr::launch_analyze(recs, n, d_workspace, (hipStream_t)stream));
    return CKR_OK;
}

}  // extern "C"

// ---- prefix-mask repair
namespace {

int repair_mantissa_bits(int dtype) {  // parse_dtype_layout (tensor_group_prefix_mask_repair.cpp:190-202)
    switch (dtype) {
        case CKR_F32: return 23;
        case CKR_F16: return 10;
        case CKR_BF16: return 7;
        default: return -1;
    }
}

// Bucket count std::unordered_map::reserve(n) gives an empty map: rehash with
// max(bucket count for 1 element, for n elements), rounded by the prime policy
// (libstdc++ bits/hashtable.h rehash, bits/hashtable_policy.h reserve).  The
// policy object is libstdc++'s own, so the numbers are the library's.
uint64_t lib_bucket_count(uint64_t n) {
    std::__detail::_Prime_rehash_policy pol;
    const size_t want = std::max<size_t>(pol._M_bkt_for_elements(1), pol._M_bkt_for_elements((size_t)n));
    return pol._M_next_bkt(want);
}

// Ascending bucket counts covering every size in [2, n]: entry j serves the
// sizes (entry j-1, entry j].
std::vector<uint64_t> bucket_table(uint64_t n) {
    std::vector<uint64_t> t;
    uint64_t lo = 2;
    for (;;) {
        const uint64_t p = lib_bucket_count(lo);
        t.push_back(p);
        if (p >= n || t.size() >= ckr::kRepairMaxPrimes) break;
        lo = p + 1;
    }
    return t;
}

struct RepairPrep {
    int es = 0;
    uint32_t k = 0;
    ckr::RepairLayout layout{};
    std::vector<uint64_t> primes;
};

int repair_prep(uint64_t n, int dtype, int masked_bits, uint32_t max_rules, bool build, RepairPrep* p) {
    const int mb = repair_mantissa_bits(dtype);
    if (mb < 0) return fail(CKR_E_INVALID, "[ckr] Unsupported dtype for mantissa-mask compression: tag %d", dtype);
    if (n >= (1ull << 31)) return fail(CKR_E_INVALID, "[ckr] repair needs n_elems < 2^31 (got %llu)", (unsigned long long)n);
    p->es = ckr_element_size(dtype);
    p->k = (uint32_t)ckr_repair_masked_bits(dtype, masked_bits);
    uint64_t nb = 1;
    if (build && n >= 2) {
        p->primes = bucket_table(n);
        nb = p->primes.back();
    }
    p->layout = ckr::repair_layout(n, p->es, p->k, max_rules, nb);
    // token ids (alphabet, then one per rule) must stay below the tombstones
    const uint32_t w = 8u * (uint32_t)p->es - p->k;
    const uint64_t ids = std::min<uint64_t>(n, 1ull << std::min<uint32_t>(w, 40)) + max_rules;
    if (ids > ckr::kRepairTomb32)
        return fail(CKR_E_INVALID, "[ckr] repair of %llu words with %u rules needs more than 32-bit token ids",
                    (unsigned long long)n, max_rules);
    return CKR_OK;
}

}  // namespace

extern "C" {

int ckr_repair_masked_bits(int dtype, int request) {
    const int mb = repair_mantissa_bits(dtype);
    if (mb < 0) return -1;
    return (request < 0 || request > mb) ? mb : request;
}

uint64_t ckr_repair_bucket_count(uint64_t n) {
    if (n < 2) return lib_bucket_count(n);
    const std::vector<uint64_t> t = bucket_table(n);
    return *std::lower_bound(t.begin(), t.end(), n);
}

uint64_t ckr_repair_workspace_bytes(uint64_t n_elems, int dtype, int masked_bits, uint32_t max_rules) {
    RepairPrep p;
    if (repair_prep(n_elems, dtype, masked_bits, max_rules, true, &p) != CKR_OK) return 0;
    return p.layout.bytes;
}

static int repair_run(const void* d_words, uint64_t n, int dtype, int masked_bits, uint32_t max_rules, bool build,
                      const ckr_repair_rule* h_rules_in, uint32_t n_rules_in, ckr_repair_rule* h_rules_out,
                      uint32_t* h_n_rules, uint64_t* h_out_tokens, uint64_t* h_max_pair, uint64_t* d_seq_out,
                      void* d_ws, uint64_t ws_bytes, void* stream) {
    RepairPrep p;
    int rc = repair_prep(n, dtype, masked_bits, build ? max_rules : n_rules_in, build, &p);
    if (rc != CKR_OK) return rc;
    if (!h_out_tokens) return fail(CKR_E_INVALID, "[ckr] null output count");
    if (build && (!h_rules_out || !h_n_rules || !h_max_pair)) return fail(CKR_E_INVALID, "[ckr] null rule outputs");
    if (!build && n_rules_in && !h_rules_in) return fail(CKR_E_INVALID, "[ckr] null rules");
    if (!build)
        for (uint32_t i = 0; i < n_rules_in; i++)
            if (h_rules_in[i].replacement != (1ull << 63) + i)
                return fail(CKR_E_INVALID, "[ckr] rule %u must have replacement 2^63 + %u", i, i);
    if (build) { *h_n_rules = 0; *h_max_pair = 0; }
    *h_out_tokens = n;
    // fewer than 2 words: no pair, no rule, nothing on the device
    // (find_best_pair returns before counting, :380-382)
    const bool trivial = build ? n < 2 : (n < 2 || n_rules_in == 0);
    hipStream_t s = (hipStream_t)stream;
    if (trivial) {
        if (d_seq_out && n) {
            // masked words as symbols: one word, or no rule to apply
            std::vector<uint64_t> h(n, 0);
            std::vector<uint8_t> raw(n * p.es);
            CKR_HIP(hipMemcpyAsync(raw.data(), d_words, raw.size(), hipMemcpyDeviceToHost, s));
            CKR_HIP(hipStreamSynchronize(s));
            const uint64_t mask = p.k ? ((1ull << p.k) - 1) : 0;
            for (uint64_t i = 0; i < n; i++) {
                uint64_t v = 0;
                std::memcpy(&v, raw.data() + i * p.es, p.es);
                h[i] = v & ~mask;
            }
            CKR_HIP(hipMemcpyAsync(d_seq_out, h.data(), n * 8, hipMemcpyHostToDevice, s));
            CKR_HIP(hipStreamSynchronize(s));
        }
        return CKR_OK;
    }
    if (!d_words) return fail(CKR_E_INVALID, "[ckr] null words");
    if (!d_ws || ws_bytes < p.layout.bytes)
        return fail(CKR_E_CAPACITY, "[ckr] repair workspace too small (%llu < %llu)", (unsigned long long)ws_bytes,
                    (unsigned long long)p.layout.bytes);
    ckr::RepairArgs a{};
    a.words = static_cast<const uint8_t*>(d_words);
    a.n = n;
    a.es = p.es;
    a.k = p.k;
    a.build = build ? 1 : 0;
    a.max_rules = build ? max_rules : n_rules_in;
    a.h_rules = h_rules_in;
    a.n_rules = n_rules_in;
    a.h_primes = p.primes.data();
    a.n_primes = (uint32_t)p.primes.size();
    a.d_seq_out = d_seq_out;
    a.recount_each_round = g_fast_paths == 0;
    a.ws = static_cast<uint8_t*>(d_ws);
    a.layout = p.layout;
    CKR_HIP(ckr::repair_launch(a, s));
    ckr::RepairCtl ctl{};
    uint8_t* ws = static_cast<uint8_t*>(d_ws);
    CKR_HIP(hipMemcpyAsync(&ctl, ws + p.layout.o_ctl, sizeof(ctl), hipMemcpyDeviceToHost, s));
    std::vector<ckr_repair_rule> rules(build ? std::max<uint32_t>(max_rules, 1) : 0);
    if (build && max_rules)
        CKR_HIP(hipMemcpyAsync(rules.data(), ws + p.layout.o_rules, sizeof(ckr_repair_rule) * max_rules,
                               hipMemcpyDeviceToHost, s));
    CKR_HIP(hipStreamSynchronize(s));
    if (ctl.err) return fail(CKR_E_CAPACITY, "[ckr] repair hash table overflow (flags %u)", ctl.err);
    *h_out_tokens = ctl.n_cur;
    if (build) {
        *h_n_rules = ctl.round;
        *h_max_pair = ctl.max_pair;
        std::memcpy(h_rules_out, rules.data(), sizeof(ckr_repair_rule) * ctl.round);
    }
    return CKR_OK;
}

int ckr_repair_build(const void* d_words, uint64_t n_elems, int dtype, int masked_bits, uint32_t max_rules,
                     ckr_repair_rule* h_rules, uint32_t* h_n_rules, uint64_t* h_out_tokens,
                     uint64_t* h_max_pair_frequency, uint64_t* d_seq_out, void* d_workspace,
                     uint64_t workspace_bytes, void* stream) {
    return repair_run(d_words, n_elems, dtype, masked_bits, max_rules, true, nullptr, 0, h_rules, h_n_rules,
                      h_out_tokens, h_max_pair_frequency, d_seq_out, d_workspace, workspace_bytes, stream);
}

int ckr_repair_apply(const void* d_words, uint64_t n_elems, int dtype, int masked_bits,
                     const ckr_repair_rule* h_rules, uint32_t n_rules, uint64_t* h_out_tokens, uint64_t* d_seq_out,
                     void* d_workspace, uint64_t workspace_bytes, void* stream) {
    return repair_run(d_words, n_elems, dtype, masked_bits, n_rules, false, h_rules, n_rules, nullptr, nullptr,
                      h_out_tokens, nullptr, d_seq_out, d_workspace, workspace_bytes, stream);
}

}  // extern "C"
