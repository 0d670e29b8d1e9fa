// checkers_amd/csrc/ckr_kernels.hip — gfx950 kernels of the checkpoint-compression path.
//
// Data layout (HBM):
//   source tensor          n_b bytes, 16-byte aligned, read with 128-bit or 32-bit loads;
//   masked byte stream     never materialised: the low `spe` bytes of every element
//                          are zeroed on load (bf16/fp16: byte 0, fp32: bytes 0-1);
//   sidecar                element-interleaved low bytes, written by the encode pass;
//   units                  the masked stream cut into `unit` bytes (multiple of 256);
//                          in a unit, lane t owns bytes t, t+256, … (256 lanes);
//   thread ↔ lanes         one thread owns the 4 lanes of one 32-bit column
//                          (lanes 4j..4j+3), so one wave64 owns one unit and each
//                          row of 256 bytes is a single coalesced 256 B load;
//   encode scratch         per unit, per lane, 32-bit slots interleaved across lanes
//                          (slot w of lane t at (w*256 + t)*4) holding the lane's
//                          output backward from its end, 4 bytes per store;
//   packed output          unit after unit, lane streams in lane order.
#include <hip/hip_runtime.h>
#include <atomic>
#include <cstdint>

#include "ckr_internal.h"
#include "ckr_table.h"

namespace ckr {

static constexpr uint32_t M = 4096u;
static constexpr uint32_t L = 1u << 23;

// ------------------------------------------------------------------ tables
// Encode entries from norm/cum (see EncSym in ckr_internal.h for the algebra).
__device__ __forceinline__ EncSym enc_entry_fc(uint32_t f, uint32_t cum) {
    EncSym e;
    if (f == 0) {
        e.rcp = 0; e.bias = 0; e.cmpl_rsh = 0; e.xmax = 0;
    } else if (f == 1) {
        e.rcp = 0xFFFFFFFFu; e.bias = cum + M - 1u; e.cmpl_rsh = (M - 1u); e.xmax = (1u << 19);
    } else {
        uint32_t l = 0;
        while ((1u << l) < f) l++;
        const uint64_t rcp = ((1ull << (31 + l)) + f - 1) / f;
        e.rcp = (uint32_t)rcp; e.bias = cum; e.cmpl_rsh = (M - f) | ((l - 1) << 16); e.xmax = f << 19;
    }
    return e;
}
__device__ __forceinline__ EncSym enc_entry(const TableArg& t, uint32_t s) { return enc_entry_fc(t.norm[s], t.cum[s]); }

// ------------------------------------------------------------------ tables on the device
// A table by ranks (ckr_table.h) in one workgroup of 256 threads, thread s for
// symbol s: the counts and their exclusive sums in LDS, the ambiguity flag.
//
// norm_fix's positions are counted by buckets of the fractional part: the
// symbols that take part in the correction (included ones, for the -1 case
// only those holding more than one slot) are counted into 256 buckets,
// bucket floor(frac * 256), whose order is that of the parts.  A symbol's
// position then lies between the count on its side of its bucket and that
// plus its bucket's count, which decides +1/-1 or 0 for every symbol except
// those of the one bucket the boundary cuts; only these compare exact parts,
// with the other members of their bucket.  Counts, ambiguity flag and sums
// equal norm_fix's over all 256 symbols.
struct RankTable {
    uint32_t norm[256], cum[257];
    double key[256];
    uint32_t bcnt[256], bpre[256];
    uint32_t blist[256];
    unsigned long long red64[4];
    uint32_t red[4], ambw[4], amb, nlist, bstar;
};

__device__ __forceinline__ uint64_t block_sum64_256(uint64_t v, unsigned long long* sh) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    return sh[0] + sh[1] + sh[2] + sh[3];
}

// Inclusive sum over the wave's lanes.
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t v) {
    const uint32_t ln = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t g = (uint32_t)__shfl_up((int)v, o, 64);
        if ((int)ln >= o) v += g;
    }
    return v;
}

// hist: read with device-scope loads (it may have been summed by other
// workgroups of the same launch).
__device__ void rank_table(const uint32_t* __restrict__ hist, bool ensure_full, RankTable& T) {
    const uint32_t s = threadIdx.x;
    const uint32_t h = __hip_atomic_load(const_cast<uint32_t*>(hist) + s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (s == 0) T.nlist = 0;
    // the total (below 2^40) and the number of symbols present, in one sum
    const uint64_t tv = block_sum64_256((uint64_t)h | ((uint64_t)(h ? 1u : 0u) << 48), T.red64);
    const uint64_t total = tv & ((1ull << 48) - 1ull), distinct = tv >> 48;
    if ((ensure_full ? 256u : distinct) == 0) {  // no symbol at all: every slot for symbol 0
        T.norm[s] = s == 0 ? kTabM : 0u;
        T.cum[s] = s == 0 ? 0u : kTabM;
        if (s == 0) { T.cum[256] = kTabM; T.amb = 0; }
        __syncthreads();
        return;
    }
    const NormStart r = norm_start(h, total, ensure_full);
    const uint32_t assigned = (uint32_t)block_sum64_256(r.norm, T.red64);
    int f = 0;
    if (assigned != kTabM) {  // (the same in every thread)
        const bool up = assigned < kTabM;
        const uint32_t rem = up ? kTabM - assigned : assigned - kTabM;
        const bool part = r.inc && (up || r.norm > 1u);
        const uint32_t b = part ? min((uint32_t)(r.frac * 256.0), 255u) : 0u;
        T.key[s] = r.frac;
        T.bcnt[s] = 0;
        __syncthreads();
        if (part) atomicAdd(&T.bcnt[b], 1u);
        __syncthreads();
        // exclusive sums over the buckets, thread s holding bucket s
        const uint32_t tsum = T.bcnt[s];
        const uint32_t inc = wave_incl_sum(tsum);
        if ((s & 63) == 63) T.red[s >> 6] = inc;
        __syncthreads();
        uint32_t pre = 0, npart = 0;
#pragma unroll
        for (uint32_t w = 0; w < 4; w++) {
            const uint32_t v = T.red[w];
            pre += w < (s >> 6) ? v : 0u;
            npart += v;
        }
        T.bpre[s] = pre + inc - tsum;
        __syncthreads();
        // up: the first rem of the descending order get +1; down: the last rem get -1.
        // lo: the symbols strictly before s on that side, counted by whole buckets
        bool need = false;
        uint32_t lo = 0;
        if (part) {
            const uint32_t below = T.bpre[b], inb = T.bcnt[b];
            lo = up ? npart - below - inb : below;
            if (lo + inb <= rem) f = up ? 1 : -1;
            else if (lo < rem) { need = true; T.bstar = b; }  // (one bucket at most)
        }
        if (__syncthreads_or(need)) {
            if (part && b == T.bstar) T.blist[atomicAdd(&T.nlist, 1u)] = s;
            __syncthreads();
            if (need) {
                const uint32_t n = T.nlist;
                uint32_t side = lo, eq = 0;
                for (uint32_t i = 0; i < n; i++) {
                    const double k = T.key[T.blist[i]];
                    side += (up ? k > r.frac : k < r.frac) ? 1u : 0u;
                    eq += k == r.frac ? 1u : 0u;
                }
                if (side + eq <= rem) f = up ? 1 : -1;
                else if (side >= rem) f = 0;
                else f = kNormAmbiguous;
            }
        }
    }
    const uint32_t nm = r.norm + (f == 1 ? 1u : 0u) - (f == -1 ? 1u : 0u);
    T.norm[s] = nm;
    // exclusive sum of the counts, the ambiguity flag beside it
    const uint32_t inc = wave_incl_sum(nm);
    const bool any_amb = __ballot(f == kNormAmbiguous) != 0;
    if ((s & 63) == 63) { T.red[s >> 6] = inc; T.ambw[s >> 6] = any_amb ? 1u : 0u; }
    __syncthreads();
    uint32_t pre = 0;
    for (uint32_t w = 0; w < (s >> 6); w++) pre += T.red[w];
    T.cum[s + 1] = pre + inc;
    if (s == 0) { T.cum[0] = 0; T.amb = (T.ambw[0] | T.ambw[1] | T.ambw[2] | T.ambw[3]) ? 1u : 0u; }
    __syncthreads();
}

// ckr_build_tables_device: one table per workgroup into a row of 258 words.
__global__ void __launch_bounds__(256) tables_kernel(const uint32_t* __restrict__ hists, int ensure_full,
                                                     uint32_t* __restrict__ rows) {
    __shared__ RankTable T;
    rank_table(hists + (uint64_t)blockIdx.x * 256, ensure_full != 0, T);
    uint32_t* row = rows + (uint64_t)blockIdx.x * 258;
    row[threadIdx.x] = T.norm[threadIdx.x];
    if (threadIdx.x == 0) { row[256] = T.cum[256]; row[257] = T.amb; }
}

// The state chains of symbol 0 for every count f in [0, 4096] (f == 0: every
// symbol the raw-byte escape), 256 steps each from state L, computed once per
// device (canon_chain_kernel, thread f): before step k, the state
// chain_x[k * kChainRows + f] and the bytes pushed so far chain_n[..]; the
// pushed bytes chain_b[j * kChainRows + f].  The canonical zero-plane streams
// of a table are then lookups instead of a serial chain.
__global__ void __launch_bounds__(256) canon_chain_kernel(uint32_t* __restrict__ chain_x, uint16_t* __restrict__ chain_n,
                                                          uint8_t* __restrict__ chain_b) {
    const uint32_t f = blockIdx.x * 256 + threadIdx.x;
    if (f >= kChainRows) return;
    const EncSym e = enc_entry_fc(f > M ? M : f, 0);
    const uint32_t rsh = e.cmpl_rsh >> 16, cm = e.cmpl_rsh & 0xFFFFu;
    uint32_t x = L, nb = 0;
    for (uint32_t k = 0; k <= kChainSteps; k++) {
        chain_x[k * kChainRows + f] = x;
        chain_n[k * kChainRows + f] = (uint16_t)nb;
        if (k == kChainSteps) break;
        if (f == 0) { chain_b[nb++ * kChainRows + f] = 0; continue; }
        const bool e1 = x >= e.xmax;
        const uint32_t x1 = e1 ? x >> 8 : x;
        const bool e2 = e1 && x1 >= e.xmax;
        if (e1) chain_b[nb++ * kChainRows + f] = (uint8_t)x;
        if (e2) chain_b[nb++ * kChainRows + f] = (uint8_t)x1;
        const uint32_t xr = e2 ? x1 >> 8 : x1;
        const uint32_t q = __umulhi(xr, e.rcp) >> rsh;
        x = xr + e.bias + __umul24(q, cm);
    }
}

struct Chains {
    const uint32_t* x;
    const uint16_t* n;
    const uint8_t* b;
};

// Canonical zero-plane streams (canon_host's layout) of lane counts K0, K1,
// K2 for symbol 0 of count f, from the state chains, in a workgroup of 256:
// canon_load issues the chain loads (used after other work), canon_put puts
// them in LDS (a barrier must follow), canon_write writes the entries: entry
// e's header {K, final state, bytes B, 0}, then its slot dwords (dword w holds
// pushed bytes 4w .. 4w+3, the first in the top byte; the last, partial one
// its r = B mod 4 bytes the same way), and after the three entries their
// streams in byte order, which are the pushed bytes reversed (stream byte q =
// pushed byte B - 1 - q).
constexpr uint32_t kPushedMax = 2 * kChainSteps + 8;  // rows of chain_b
struct CanonLds {
    uint32_t ex[3], eb[3];
    uint8_t pb[kPushedMax];
};
struct CanonLoad {
    uint8_t b0, b1, b2;
    uint32_t exv, ebv;
};
__device__ __forceinline__ CanonLoad canon_load(uint32_t f, uint32_t k0, uint32_t k1, uint32_t k2, const Chains& ch) {
    const uint32_t s = threadIdx.x;
    const uint32_t kmax = min(max(k0, max(k1, k2)), kChainSteps);
    const uint32_t npb = 2 * kmax + 8;  // at least the bytes pushed in kmax steps
    CanonLoad c{0, 0, 0, 0u, 0u};
    if (s < npb) c.b0 = ch.b[s * kChainRows + f];
    if (s + 256 < npb) c.b1 = ch.b[(s + 256) * kChainRows + f];
    if (s + 512 < npb) c.b2 = ch.b[(s + 512) * kChainRows + f];
    if (s < 3) {
        const uint32_t K = s == 0 ? k0 : (s == 1 ? k1 : k2);
        c.exv = ch.x[K * kChainRows + f];
        c.ebv = ch.n[K * kChainRows + f];
    }
    return c;
}
__device__ __forceinline__ void canon_put(const CanonLoad& c, CanonLds& C) {
    const uint32_t s = threadIdx.x;
    C.pb[s] = c.b0;
    if (s + 256 < kPushedMax) C.pb[s + 256] = c.b1;
    if (s + 512 < kPushedMax) C.pb[s + 512] = c.b2;
    if (s < 3) { C.ex[s] = c.exv; C.eb[s] = c.ebv; }
}
__device__ __forceinline__ void canon_write(uint32_t k0, uint32_t k1, uint32_t k2, uint32_t cw, const CanonLds& C,
                                            uint32_t* __restrict__ canon) {
    const uint32_t s = threadIdx.x;
    for (uint32_t en = 0; en < 3; en++) {
        const uint32_t B = C.eb[en], w = B >> 2, r = B & 3u;
        for (uint32_t d = s; d < cw; d += 256) {
            uint32_t sv = 0;
            if (d < w) sv = ((uint32_t)C.pb[4 * d] << 24) | ((uint32_t)C.pb[4 * d + 1] << 16) | ((uint32_t)C.pb[4 * d + 2] << 8) | C.pb[4 * d + 3];
            else if (d == w) for (uint32_t i = 0; i < r; i++) sv = (sv << 8) | C.pb[4 * w + i];
            uint32_t bv = 0;
#pragma unroll
            for (uint32_t k = 0; k < 4; k++) {
                const uint32_t q = 4 * d + k;
                if (q < B) bv |= (uint32_t)C.pb[B - 1 - q] << (8 * k);
            }
            canon[en * (4 + cw) + 4 + d] = sv;
            canon[3 * (4 + cw) + en * cw + d] = bv;
        }
    }
    if (s < 3) {
        uint32_t* base = canon + s * (4 + cw);
        base[0] = s == 0 ? k0 : (s == 1 ? k1 : k2);
        base[1] = C.ex[s];
        base[2] = C.eb[s];
        base[3] = 0;
    }
}

// LDS of table_enc_body (the histogram kernel's copies, reused once they are
// summed).
struct TableLds {
    RankTable T;
    float fred[4][8];
    CanonLds C;
};

// The encode set-up of a tensor from its histograms on the device (no host
// round trip): the table by ranks, the encode entries, the canonical
// zero-plane streams, the fast encoder's LDS slot sizes, and its control words
// cleared.  tinfo: norm[256], sum, ambiguity flag, slot bytes of the two live
// planes.  The slot sizes follow lane_slot_bytes on the host (expected coded
// size of K symbols from the plane histograms plus six standard deviations),
// then the larger is cut until both fit the launch's LDS (sum at most 2 smax).
// ctl[6..7] gets the launch's epoch, the sign for the host that the table was
// built in this launch; ctl[2] (failure flags) starts as flags.  The
// canonical streams are those of symbol 0 of count f = norm[0].
__device__ void table_enc_body(const uint32_t* __restrict__ hist, const TableEncArg& a, EncSym* __restrict__ enc,
                               uint32_t* __restrict__ canon, uint32_t* __restrict__ tinfo, uint32_t* __restrict__ ctl,
                               const Chains& ch, uint64_t epoch, uint32_t flags, TableLds& W) {
    RankTable& T = W.T;
    rank_table(hist, a.ensure_full != 0, T);
    const uint32_t s = threadIdx.x;
    // the chain data of the canonical streams, loaded now and used at the end
    const CanonLoad cl = canon_load(T.norm[0], a.k0, a.k1, a.k2, ch);
    const uint32_t nm = T.norm[s];
    enc[s] = enc_entry_fc(nm, T.cum[s]);
    tinfo[s] = nm;
    if (s < 6) ctl[s] = s == 2 ? flags : 0u;
    // slot sizes: per plane p, n = sum h_p, m = sum h_p cost / n, v = sum h_p cost^2 / n - m^2
    const float cost = nm ? 12.0f - log2f((float)nm) : 8.0f;  // log2(M / norm)
    float v[6];
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const float hp = (float)__hip_atomic_load(const_cast<uint32_t*>(hist) + 256 + 256 * p + s, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        v[3 * p] = hp;
        v[3 * p + 1] = hp * cost;
        v[3 * p + 2] = hp * cost * cost;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int i = 0; i < 6; i++) v[i] += __shfl_xor(v[i], o, 64);
    if ((s & 63) == 0)
#pragma unroll
        for (int i = 0; i < 6; i++) W.fred[s >> 6][i] = v[i];
    canon_put(cl, W.C);
    __syncthreads();
    if (s == 0) {
        uint32_t sl[2];
        for (int p = 0; p < 2; p++) {
            const double cnt = (double)W.fred[0][3 * p] + W.fred[1][3 * p] + W.fred[2][3 * p] + W.fred[3][3 * p];
            if (cnt <= 0.0) { sl[p] = 8; continue; }
            const double s1 = (double)W.fred[0][3 * p + 1] + W.fred[1][3 * p + 1] + W.fred[2][3 * p + 1] + W.fred[3][3 * p + 1];
            const double s2 = (double)W.fred[0][3 * p + 2] + W.fred[1][3 * p + 2] + W.fred[2][3 * p + 2] + W.fred[3][3 * p + 2];
            const double mean = s1 / cnt, var = fmax(s2 / cnt - mean * mean, 0.0);
            const double bits = a.K * mean + 6.0 * sqrt(a.K * var) + 32.0;
            uint64_t bytes = (uint64_t)ceil(bits / 8.0) + 8;
            bytes = (bytes + 3) & ~3ull;
            bytes = bytes < 8 ? 8 : bytes;
            sl[p] = (uint32_t)(bytes < 2ull * a.K + 8 ? bytes : 2ull * a.K + 8);
        }
        while (sl[0] + sl[1] > 2 * a.smax && (sl[0] > 8 || sl[1] > 8)) (sl[0] >= sl[1] ? sl[0] : sl[1]) -= 4;
        tinfo[256] = T.cum[256];
        tinfo[257] = T.amb;
        tinfo[258] = sl[0];
        tinfo[259] = sl[1];
        ctl[6] = (uint32_t)epoch;
        ctl[7] = (uint32_t)(epoch >> 32);
    }
    canon_write(a.k0, a.k1, a.k2, a.cw, W.C, canon);
}

__global__ void __launch_bounds__(256) build_enc_table_kernel(TableArg t, EncSym* out) {
    out[threadIdx.x] = enc_entry(t, threadIdx.x);
}

// The fast encoder's set-up in one launch: the encode entries (block 0), its
// look-back status words cleared, and its control words (ctl[0]: ticket
// counter, ctl[1]: redo-list length, ctl[2]: failure flags, ctl[3]: the redo
// launch's ticket counter, ctl[4..5]: the packed total, written with the last
// unit's offset) cleared.
__global__ void __launch_bounds__(256) build_enc_table_reset_kernel(TableArg t, EncSym* out, uint64_t* status,
                                                                    uint64_t n, uint32_t* ctl) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blockIdx.x == 0) {
        out[threadIdx.x] = enc_entry(t, threadIdx.x);
        if (threadIdx.x < 6) ctl[threadIdx.x] = 0;
    }
    if (i < n) status[i] = 0;
}

// Decode slots from norm/cum: slot j in [cum[s], cum[s]+norm[s]) → s.  One
// thread per slot (16 blocks of 256): the symbol is the last s with cum[s] <= j
// and norm[s] > 0, found by binary search over the prefix sums.  bad (when not
// null): the decoder's bad-lane counter, cleared here for the launch after.
__global__ void __launch_bounds__(256) build_dec_table_kernel(TableArg t, uint32_t* out, unsigned long long* bad) {
    if (bad && blockIdx.x == 0 && threadIdx.x == 0) *bad = 0;
    __shared__ uint32_t cum[257];
    for (uint32_t i = threadIdx.x; i < 257; i += 256) cum[i] = t.cum[i];
    __syncthreads();
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    // largest s with cum[s] <= j < cum[s+1] (empty symbols have cum[s] == cum[s+1])
    uint32_t lo = 0, hi = 256;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (cum[mid] <= j) lo = mid; else hi = mid;
    }
    const uint32_t f = t.norm[lo];
    if (j < cum[256] && f) out[j] = lo | ((f - 1u) << 8) | (cum[lo] << 20);
}

// ------------------------------------------------------------------ byte-plane split
template <int SPE>
__device__ __forceinline__ uint32_t live_mask32() {
    return SPE == 2 ? 0xFFFF0000u : (SPE == 1 ? 0xFF00FF00u : 0xFFFFFFFFu);
}
__device__ __forceinline__ bool byte_live(uint64_t pos, int es, int spe) {
    return (int)(pos % (uint64_t)es) >= spe;
}

// 128-bit loads; masked = src & live mask, sidecar gathered per element.
template <int SPE>
__global__ void __launch_bounds__(256) extract_mantissa_kernel(const uint8_t* __restrict__ src,
                                                               uint64_t n_bytes,
                                                               uint8_t* __restrict__ masked,
                                                               uint8_t* __restrict__ sidecar) {
    const uint64_t nvec = n_bytes / 16;
    const uint32_t lm = live_mask32<SPE>();
    for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec;
         v += (uint64_t)gridDim.x * blockDim.x) {
        uint4 x = reinterpret_cast<const uint4*>(src)[v];
        reinterpret_cast<uint4*>(masked)[v] = make_uint4(x.x & lm, x.y & lm, x.z & lm, x.w & lm);
        if (SPE == 2) {  // 4 fp32 elements → 8 sidecar bytes
            uint2 sc;
            sc.x = (x.x & 0xFFFFu) | (x.y << 16);
            sc.y = (x.z & 0xFFFFu) | (x.w << 16);
            reinterpret_cast<uint2*>(sidecar)[v] = sc;
        } else {         // 8 two-byte elements → 8 sidecar bytes (byte 0 of each)
            uint2 sc;
            sc.x = (x.x & 0xFFu) | ((x.x >> 8) & 0xFF00u) | ((x.y & 0xFFu) << 16) | ((x.y >> 16) & 0xFFu) << 24;
            sc.y = (x.z & 0xFFu) | ((x.z >> 8) & 0xFF00u) | ((x.w & 0xFFu) << 16) | ((x.w >> 16) & 0xFFu) << 24;
            reinterpret_cast<uint2*>(sidecar)[v] = sc;
        }
    }
    // tail bytes (fewer than 16)
    if (blockIdx.x == 0) {
        const int es = SPE == 2 ? 4 : 2;
        for (uint64_t p = nvec * 16 + threadIdx.x; p < n_bytes; p += blockDim.x) {
            const uint8_t b = src[p];
            const int plane = (int)(p % es);
            masked[p] = plane < SPE ? 0 : b;
            if (plane < SPE) sidecar[(p / es) * SPE + plane] = b;
        }
    }
}

// The same split one byte per thread, for buffers that are only element-aligned.
template <int SPE>
__global__ void __launch_bounds__(256) extract_mantissa_bytes_kernel(const uint8_t* __restrict__ src,
                                                                     uint64_t n_bytes,
                                                                     uint8_t* __restrict__ masked,
                                                                     uint8_t* __restrict__ sidecar) {
    constexpr int es = SPE == 2 ? 4 : 2;
    for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < n_bytes;
         p += (uint64_t)gridDim.x * blockDim.x) {
        const uint8_t b = src[p];
        const int plane = (int)(p % es);
        masked[p] = plane < SPE ? 0 : b;
        if (plane < SPE) sidecar[(p / es) * SPE + plane] = b;
    }
}

hipError_t launch_extract_mantissa(const uint8_t* src, uint64_t n_elems, int es, int spe,
                                   uint8_t* masked, uint8_t* sidecar, hipStream_t s) {
    const uint64_t n_bytes = n_elems * (uint64_t)es;
    const uint64_t nvec = n_bytes / 16;
    uint32_t grid = (uint32_t)std::min<uint64_t>((nvec + 255) / 256, 8192);
    if (grid == 0) grid = 1;
    const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(masked) |
                       reinterpret_cast<uintptr_t>(sidecar)) & 15u) == 0;
    if (!vec) {
        grid = (uint32_t)std::min<uint64_t>((n_bytes + 255) / 256, 8192);
        if (grid == 0) grid = 1;
        if (spe == 2) CKR_LAUNCH("extract_mantissa_bytes_kernel", s, extract_mantissa_bytes_kernel<2><<<grid, 256, 0, s>>>(src, n_bytes, masked, sidecar));
        else CKR_LAUNCH("extract_mantissa_bytes_kernel", s, extract_mantissa_bytes_kernel<1><<<grid, 256, 0, s>>>(src, n_bytes, masked, sidecar));
        return hipGetLastError();
    }
    if (spe == 2) CKR_LAUNCH("extract_mantissa_kernel", s, extract_mantissa_kernel<2><<<grid, 256, 0, s>>>(src, n_bytes, masked, sidecar));
    else CKR_LAUNCH("extract_mantissa_kernel", s, extract_mantissa_kernel<1><<<grid, 256, 0, s>>>(src, n_bytes, masked, sidecar));
    return hipGetLastError();
}

// ------------------------------------------------------------------ masked histogram
// 32 bank-interleaved LDS copies (bin b of copy c at b*32 + c, copy = lane & 31),
// so the ds_add of a wave never hits the same bank twice whatever the data; the
// zero planes are not counted here (their count, n_elems*spe, is put in bin 0
// by the init kernel).  Each block adds its 256 sums to the global histogram
// with integer atomics (order-independent, so the result is deterministic).
static constexpr uint32_t HIST_COPIES = 32;

// LDS slot of a count: raw dtypes 32 copies of one histogram; masked dtypes PC
// copies of each of the two live planes (rank 0: byte 2 of fp32 / byte 1 of a
// 16-bit pair, rank 1: byte 3), so per-plane histograms come for free.
template <int SPE, int PC = 16>
__device__ __forceinline__ uint32_t hist_slot(uint32_t bin, uint32_t rank, uint32_t c) {
    if (SPE == 0) return bin * HIST_COPIES + c;
    return (rank * 256 + bin) * PC + (c & (PC - 1));
}

template <int SPE, int PC = 16>
__device__ __forceinline__ void hist_add_dword(uint32_t* sh, uint32_t v, uint32_t c) {
#pragma unroll
    for (int b = 0; b < 4; b++) {
        if (SPE == 2 && b < 2) continue;
        if (SPE == 1 && (b & 1) == 0) continue;
        atomicAdd(&sh[hist_slot<SPE, PC>((v >> (8 * b)) & 255u, b == 3 ? 1u : 0u, c)], 1u);
    }
}

// hist[256]: total, the zero planes counted in closed form into bin 0;
// planes[512] (optional, masked dtypes): the two live planes.
// ctr (optional): masked_hist_chunks_kernel's chunk counter.
__global__ void __launch_bounds__(256) hist_init_kernel(uint32_t* __restrict__ hist, uint64_t zero_count,
                                                        uint32_t* __restrict__ planes, uint32_t* __restrict__ ctr) {
    hist[threadIdx.x] = (threadIdx.x == 0) ? (uint32_t)zero_count : 0u;
    if (planes) { planes[threadIdx.x] = 0; planes[256 + threadIdx.x] = 0; }
    if (ctr && threadIdx.x == 0) *ctr = 0;
}

// PC: copies per live plane (masked dtypes).  16 (32 KiB of LDS) when the
// kernel has the device to itself; 4 (8 KiB) when it runs beside the fast
// encoder, whose workgroup leaves about 10 KiB of a CU's LDS free.
//
// src is 16-byte aligned; the head_n (< 16) bytes before it, at src - head_n,
// are the tensor's first bytes when the tensor itself is only element-aligned
// (head_n is then a multiple of the element size, so every byte keeps its
// plane).  Positions below are counted from src; a head byte at src - head_n +
// i is at position i - head_n.
// One workgroup's share (block b of nb) of one tensor's histogram, added into
// hist (and planes) at the end; sh: the workgroup's LDS copies.
//
// gate (hist_table_kernel): the sums are added only once *gate holds epoch, the
// sign that the job's first workgroup has cleared hist; a wait that outlasts
// kGateSpins polls skips the adds and stores epoch in *gate_err instead.
constexpr uint32_t kGateSpins = 1u << 22;
// Pieces of a workgroup's histogram pass (sh: its PC copies per live plane,
// c: this thread's copy): the bytes before the 16-byte aligned start (head_n,
// at src - head_n), the 16-byte vectors [v, end) with stride, the bytes after
// the last whole vector, and the sums added to the global counters.
template <int SPE, int PC>
__device__ __forceinline__ void hist_head_bytes(uint32_t* sh, const uint8_t* __restrict__ src, int es, uint32_t head_n,
                                                uint32_t c) {
    if (threadIdx.x < head_n) {
        const int64_t p = (int64_t)threadIdx.x - (int64_t)head_n;
        const int plane = (int)(((p % es) + es) % es);
        if (plane >= SPE) {
            const uint32_t r = (SPE > 0 && (p & 3) == 3) ? 1u : 0u;
            atomicAdd(&sh[hist_slot<SPE, PC>((uint32_t)src[p], r, c)], 1u);
        }
    }
}
template <int SPE, int PC>
__device__ __forceinline__ void hist_vectors(uint32_t* sh, const uint4* __restrict__ v4, uint64_t v, uint64_t end,
                                             uint64_t stride, uint32_t c) {
    for (; v + 3 * stride < end; v += 4 * stride) {  // 4 loads in flight per thread
        uint4 a = v4[v], b = v4[v + stride], d = v4[v + 2 * stride], e = v4[v + 3 * stride];
        hist_add_dword<SPE, PC>(sh, a.x, c); hist_add_dword<SPE, PC>(sh, a.y, c);
        hist_add_dword<SPE, PC>(sh, a.z, c); hist_add_dword<SPE, PC>(sh, a.w, c);
        hist_add_dword<SPE, PC>(sh, b.x, c); hist_add_dword<SPE, PC>(sh, b.y, c);
        hist_add_dword<SPE, PC>(sh, b.z, c); hist_add_dword<SPE, PC>(sh, b.w, c);
        hist_add_dword<SPE, PC>(sh, d.x, c); hist_add_dword<SPE, PC>(sh, d.y, c);
        hist_add_dword<SPE, PC>(sh, d.z, c); hist_add_dword<SPE, PC>(sh, d.w, c);
        hist_add_dword<SPE, PC>(sh, e.x, c); hist_add_dword<SPE, PC>(sh, e.y, c);
        hist_add_dword<SPE, PC>(sh, e.z, c); hist_add_dword<SPE, PC>(sh, e.w, c);
    }
    for (; v < end; v += stride) {
        uint4 a = v4[v];
        hist_add_dword<SPE, PC>(sh, a.x, c); hist_add_dword<SPE, PC>(sh, a.y, c);
        hist_add_dword<SPE, PC>(sh, a.z, c); hist_add_dword<SPE, PC>(sh, a.w, c);
    }
}
template <int SPE, int PC>
__device__ __forceinline__ void hist_tail_bytes(uint32_t* sh, const uint8_t* __restrict__ src, uint64_t n_bytes, int es,
                                                uint32_t c) {
    for (uint64_t p = (n_bytes / 16) * 16 + threadIdx.x; p < n_bytes; p += blockDim.x) {
        const int plane = (int)(p % (uint64_t)es);
        if (plane < SPE) continue;
        const uint32_t r = (SPE > 0 && (p & 3) == 3) ? 1u : 0u;  // live-plane rank
        atomicAdd(&sh[hist_slot<SPE, PC>((uint32_t)src[p], r, c)], 1u);
    }
}
template <int SPE, int PC>
__device__ __forceinline__ void hist_flush(const uint32_t* sh, uint32_t* __restrict__ hist, uint32_t* __restrict__ planes) {
    const uint32_t bin = threadIdx.x;
    if (SPE == 0) {
        uint32_t sum = 0;
#pragma unroll 8
        for (uint32_t k = 0; k < HIST_COPIES; k++) sum += sh[bin * HIST_COPIES + ((k + bin) & (HIST_COPIES - 1))];
        if (sum) atomicAdd(&hist[bin], sum);
    } else {
        uint32_t s0 = 0, s1 = 0;
#pragma unroll 8
        for (uint32_t k = 0; k < (uint32_t)PC; k++) {
            s0 += sh[hist_slot<SPE, PC>(bin, 0, (k + bin) & (PC - 1))];
            s1 += sh[hist_slot<SPE, PC>(bin, 1, (k + bin) & (PC - 1))];
        }
        if (s0 + s1) atomicAdd(&hist[bin], s0 + s1);
        if (planes) {  // per live plane, rank 0 / rank 1
            if (s0) atomicAdd(&planes[bin], s0);
            if (s1) atomicAdd(&planes[256 + bin], s1);
        }
    }
}

template <int SPE, int PC>
__device__ __forceinline__ void masked_hist_share(uint32_t* sh, const uint8_t* __restrict__ src, uint64_t n_bytes,
                                                  int es, uint32_t* __restrict__ hist, uint32_t* __restrict__ planes,
                                                  uint32_t head_n, uint32_t b, uint32_t nb,
                                                  unsigned long long* gate = nullptr, unsigned long long epoch = 0,
                                                  unsigned long long* gate_err = nullptr) {
    constexpr uint32_t NSH = SPE == 0 ? 256 * HIST_COPIES : 512 * PC;
    for (uint32_t i = threadIdx.x; i < NSH; i += blockDim.x) sh[i] = 0;
    __syncthreads();
    const uint32_t c = threadIdx.x & (HIST_COPIES - 1);
    if (b == 0) hist_head_bytes<SPE, PC>(sh, src, es, head_n, c);
    const uint64_t stride = (uint64_t)nb * blockDim.x;
    hist_vectors<SPE, PC>(sh, reinterpret_cast<const uint4*>(src), (uint64_t)b * blockDim.x + threadIdx.x, n_bytes / 16,
                          stride, c);
    if (b == 0) hist_tail_bytes<SPE, PC>(sh, src, n_bytes, es, c);
    if (gate) {
        __shared__ uint32_t open;
        if (threadIdx.x == 0) {
            uint32_t n = 0;
            // relaxed polls (an acquire would invalidate the L2 at every poll): the
            // adds after the loop are device-scope atomics and need no acquire
            while (__hip_atomic_load(gate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch && ++n < kGateSpins)
                __builtin_amdgcn_s_sleep(2);
            open = n < kGateSpins;
            if (!open) __hip_atomic_store(gate_err, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!open) return;
    }
    __syncthreads();
    hist_flush<SPE, PC>(sh, hist, planes);
}

template <int SPE, int PC>
__global__ void __launch_bounds__(256) masked_hist_kernel(const uint8_t* __restrict__ src, uint64_t n_bytes,
                                                          int es, uint32_t* __restrict__ hist,
                                                          uint32_t* __restrict__ planes, uint32_t head_n) {
    __shared__ uint32_t sh[SPE == 0 ? 256 * HIST_COPIES : 512 * PC];
    masked_hist_share<SPE, PC>(sh, src, n_bytes, es, hist, planes, head_n, blockIdx.x, gridDim.x);
}

// The histogram beside a running encoder (PC copies per plane), its
// workgroups taking chunks of kHistChunkVecs vectors from a counter (*ctr,
// cleared by hist_init_kernel) instead of fixed shares.  Beside the encoder one
// workgroup fits per CU; as the encoder's workgroups leave their CUs the
// grid's other workgroups are dispatched there and join in, so that the pass
// finishes at full width instead of on one workgroup per CU.  The workgroup
// that first finds the chunks gone counts the head and tail bytes; a
// workgroup that counted nothing adds nothing.
constexpr uint64_t kHistChunkVecs = 16384;  // 256 KiB
template <int SPE, int PC>
__global__ void __launch_bounds__(256) masked_hist_chunks_kernel(const uint8_t* __restrict__ src, uint64_t n_bytes,
                                                                 int es, uint32_t* __restrict__ hist,
                                                                 uint32_t* __restrict__ planes, uint32_t head_n,
                                                                 uint32_t* __restrict__ ctr) {
    __shared__ uint32_t sh[SPE == 0 ? 256 * HIST_COPIES : 512 * PC];
    __shared__ uint32_t ticket;
    constexpr uint32_t NSH = SPE == 0 ? 256 * HIST_COPIES : 512 * PC;
    for (uint32_t i = threadIdx.x; i < NSH; i += blockDim.x) sh[i] = 0;
    const uint32_t c = threadIdx.x & (HIST_COPIES - 1);
    const uint64_t nvec = n_bytes / 16;
    const uint64_t nch = (nvec + kHistChunkVecs - 1) / kHistChunkVecs;
    bool counted = false;
    for (;;) {
        __syncthreads();
        if (threadIdx.x == 0) ticket = atomicAdd(ctr, 1u);
        __syncthreads();
        const uint64_t k = ticket;
        if (k >= nch) {
            if (k == nch) {  // (one workgroup)
                hist_head_bytes<SPE, PC>(sh, src, es, head_n, c);
                hist_tail_bytes<SPE, PC>(sh, src, n_bytes, es, c);
                counted = true;
            }
            break;
        }
        counted = true;
        const uint64_t v0 = k * kHistChunkVecs, v1 = v0 + kHistChunkVecs < nvec ? v0 + kHistChunkVecs : nvec;
        hist_vectors<SPE, PC>(sh, reinterpret_cast<const uint4*>(src), v0 + threadIdx.x, v1, blockDim.x, c);
    }
    __syncthreads();
    if (counted) hist_flush<SPE, PC>(sh, hist, planes);
}

// Several tensors' histograms in one grid (ckr_compress_many on a shard of
// small tensors): block b works for the last job whose first block is <= b.
// Each job's 768 words (histogram, then the two live planes') are set up by
// hist_init_multi_kernel, one block per job, before it.
__global__ void __launch_bounds__(256) hist_init_multi_kernel(HistJobs jobs) {
    const HistJob& j = jobs.j[blockIdx.x];
    for (uint32_t i = threadIdx.x; i < 768; i += blockDim.x) j.hist[i] = (i == 0) ? (uint32_t)j.zero_count : 0u;
}

__global__ void __launch_bounds__(256) masked_hist_multi_kernel(HistJobs jobs) {
    __shared__ uint32_t sh[256 * HIST_COPIES];  // = 512 x 16, the masked dtypes' copies
    uint32_t k = 0;
    while (k + 1 < jobs.n && jobs.j[k + 1].blk0 <= blockIdx.x) k++;
    const HistJob& j = jobs.j[k];
    const uint32_t b = blockIdx.x - j.blk0;
    if (j.spe == 2) masked_hist_share<2, 16>(sh, j.src, j.n_bytes, j.es, j.hist, j.hist + 256, j.head_n, b, j.nblk);
    else if (j.spe == 1) masked_hist_share<1, 16>(sh, j.src, j.n_bytes, j.es, j.hist, j.hist + 256, j.head_n, b, j.nblk);
    else masked_hist_share<0, 16>(sh, j.src, j.n_bytes, j.es, j.hist, nullptr, j.head_n, b, j.nblk);
}

// Histograms and encode set-ups of up to kMaxHistJobs masked tensors in one
// grid (launch_hist_table).  Job k's workgroups (blk0 .. blk0 + nblk): the
// first clears the job's histogram words and done counter, then opens the
// job's gate with the launch's epoch (no earlier launch used that value, so
// whatever the words held before cannot open it); each counts its share into
// LDS, adds its sums once the gate is open, and takes a done ticket; the one
// that takes the last ticket builds the table in the same LDS
// (table_enc_body).  Every workgroup also clears a share of the job's
// look-back status words.  Words of hist: 768 counts, gate (768-769), done
// counter (770), gate time-out stamp (772-773).
struct HistTableJob {
    HistJob h;
    TableEncJob t;
};
struct HistTableJobs {
    uint32_t n;
    unsigned long long epoch;
    HistTableJob j[kMaxHistJobs];
};
__global__ void __launch_bounds__(256) hist_table_kernel(HistTableJobs J, Chains ch) {
    __shared__ __align__(16) uint32_t sh[512 * 16];
    static_assert(sizeof(TableLds) <= sizeof(sh), "the table set-up reuses the histogram's LDS");
    __shared__ uint32_t last;
    uint32_t k = 0;
    while (k + 1 < J.n && J.j[k + 1].h.blk0 <= blockIdx.x) k++;
    const HistJob& j = J.j[k].h;
    const TableEncJob& t = J.j[k].t;
    const uint32_t b = blockIdx.x - j.blk0;
    auto* gate = reinterpret_cast<unsigned long long*>(j.hist + 768);
    auto* gate_err = reinterpret_cast<unsigned long long*>(j.hist + 772);
    uint32_t* done = j.hist + 770;
    for (uint64_t i = (uint64_t)b * 256 + threadIdx.x; i < t.n_status; i += (uint64_t)j.nblk * 256) t.status[i] = 0;
    if (b == 0) {  // device-scope stores, complete (s_waitcnt) before the gate opens
        for (uint32_t i = threadIdx.x; i < 768; i += 256)
            __hip_atomic_store(j.hist + i, i == 0 ? (uint32_t)j.zero_count : 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (threadIdx.x == 0) __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_store(gate, J.epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (j.spe == 2)
        masked_hist_share<2, 16>(sh, j.src, j.n_bytes, j.es, j.hist, j.hist + 256, j.head_n, b, j.nblk, gate, J.epoch, gate_err);
    else
        masked_hist_share<1, 16>(sh, j.src, j.n_bytes, j.es, j.hist, j.hist + 256, j.head_n, b, j.nblk, gate, J.epoch, gate_err);
    // this workgroup's adds complete (every wave waits for its own) before its
    // ticket; the table reads the counts with device-scope loads
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == j.nblk - 1;
    __syncthreads();
    if (!last) return;
    const uint32_t flags = __hip_atomic_load(gate_err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == J.epoch ? 4u : 0u;
    table_enc_body(j.hist, t.a, t.enc, t.canon, t.tinfo, t.ctl, ch, J.epoch, flags, *reinterpret_cast<TableLds*>(sh));
}


// Every workgroup ends with up to 768 global atomics (the sums of its LDS
// copies), so the grid is kept small: 256 workgroups (one per CU) below 256
// MiB, 512 above.  Measured on MI355X for a 4 GB fp32 tensor: 0.69 ms with 512
// workgroups, 0.77 ms with 2048; for a 64 MiB one 17 us with 256, 46 us with
// 2048.
uint32_t hist_num_blocks(uint64_t n_bytes) {
    const uint64_t nvec = n_bytes / 16;
    uint64_t nb = (nvec + 1023) / 1024;  // >= 4 vectors per thread
    const uint64_t cap = nvec >= (16ull << 20) ? 512 : 256;
    if (nb < 1) nb = 1;
    if (nb > cap) nb = cap;
    return (uint32_t)nb;
}

hipError_t launch_masked_hist(const uint8_t* src, uint64_t n_bytes, int es, int spe, uint32_t* d_hist,
                              uint32_t* d_planes, hipStream_t s, bool lean, uint32_t* chunk_ctr) {
    const uint64_t zero_count = (es > 0) ? (n_bytes / (uint64_t)es) * (uint64_t)spe : 0;
    if (spe == 0) d_planes = nullptr;
    if (!lean || spe == 0) chunk_ctr = nullptr;
    CKR_LAUNCH("hist_init_kernel", s, hist_init_kernel<<<1, 256, 0, s>>>(d_hist, zero_count, d_planes, chunk_ctr));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (n_bytes == 0) return hipSuccess;
    // an element-aligned source: its bytes up to the next 16-byte boundary are
    // counted one at a time, the rest with 16-byte loads
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(src) & 15u);
    const uint32_t head_n = (uint32_t)std::min<uint64_t>(mis ? 16u - mis : 0u, n_bytes);
    src += head_n;
    n_bytes -= head_n;
    uint32_t nblk = hist_num_blocks(n_bytes);
    if (lean) {
        // one workgroup per CU: beside a running encoder the pass then takes
        // about the encoder's spare HBM bandwidth; at full width it takes all of
        // it and the latency-bound encoder slows by as much as the pass saves
        int dev = 0, ncu = 0;
        if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
        if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
        if (ncu > 0 && nblk > (uint32_t)ncu) nblk = (uint32_t)ncu;
        if (chunk_ctr) {  // chunks from a counter (launch_masked_hist_join can add workgroups)
            const uint32_t grid = (uint32_t)std::max(ncu, 1);
            if (spe == 2)
                CKR_LAUNCH("masked_hist_kernel", s, masked_hist_chunks_kernel<2, 4><<<grid, 256, 0, s>>>(src, n_bytes, es, d_hist, d_planes, head_n, chunk_ctr));
            else
                CKR_LAUNCH("masked_hist_kernel", s, masked_hist_chunks_kernel<1, 4><<<grid, 256, 0, s>>>(src, n_bytes, es, d_hist, d_planes, head_n, chunk_ctr));
            return hipGetLastError();
        }
    }
    auto run = [&](auto kern) {
        CKR_LAUNCH("masked_hist_kernel", s, kern<<<nblk, 256, 0, s>>>(src, n_bytes, es, d_hist, d_planes, head_n));
    };
    if (spe == 2) lean ? run(masked_hist_kernel<2, 4>) : run(masked_hist_kernel<2, 16>);
    else if (spe == 1) lean ? run(masked_hist_kernel<1, 4>) : run(masked_hist_kernel<1, 16>);
    else run(masked_hist_kernel<0, 16>);
    return hipGetLastError();
}

// Workgroup shares of a set of histogram jobs: about 512 in all, in proportion
// to their bytes, at least one each and never more than a lone launch would
// take (every workgroup ends with up to 768 global atomics).
static uint32_t hist_shares(const HistSrc* srcs, uint32_t n, HistJob* out, uint32_t* const* hists) {
    uint64_t total = 0;
    for (uint32_t k = 0; k < n; k++) total += srcs[k].n_bytes;
    uint32_t nb = 0;
    for (uint32_t k = 0; k < n; k++) {
        const HistSrc& x = srcs[k];
        HistJob& j = out[k];
        const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(x.src) & 15u);
        j.head_n = (uint32_t)std::min<uint64_t>(mis ? 16u - mis : 0u, x.n_bytes);
        j.src = x.src + j.head_n;
        j.n_bytes = x.n_bytes - j.head_n;
        j.es = x.es;
        j.spe = x.spe;
        j.zero_count = (x.es > 0) ? (x.n_bytes / (uint64_t)x.es) * (uint64_t)x.spe : 0;
        j.hist = hists[k];
        const uint64_t share = total ? (512ull * x.n_bytes + total - 1) / total : 1;
        j.nblk = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(share, hist_num_blocks(j.n_bytes)));
        j.blk0 = nb;
        nb += j.nblk;
    }
    return nb;
}
hipError_t launch_masked_hist_join(const uint8_t* src, uint64_t n_bytes, int es, int spe, uint32_t* d_hist,
                                   uint32_t* d_planes, uint32_t* chunk_ctr, uint32_t per_cu, hipStream_t s) {
    if (spe != 1 && spe != 2) return hipErrorInvalidValue;
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(src) & 15u);
    const uint32_t head_n = (uint32_t)std::min<uint64_t>(mis ? 16u - mis : 0u, n_bytes);
    int dev = 0, ncu = 0;
    hipError_t e;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    const uint32_t grid = per_cu * (uint32_t)std::max(ncu, 1);
    // full-width copies (16 per plane): these workgroups run once the CUs are free
    if (spe == 2)
        CKR_LAUNCH("masked_hist_kernel", s, masked_hist_chunks_kernel<2, 16><<<grid, 256, 0, s>>>(src + head_n, n_bytes - head_n, es, d_hist, d_planes, head_n, chunk_ctr));
    else
        CKR_LAUNCH("masked_hist_kernel", s, masked_hist_chunks_kernel<1, 16><<<grid, 256, 0, s>>>(src + head_n, n_bytes - head_n, es, d_hist, d_planes, head_n, chunk_ctr));
    return hipGetLastError();
}

hipError_t launch_masked_hist_multi(const HistSrc* srcs, uint32_t n, uint32_t* d_hists, hipStream_t s) {
    for (uint32_t j0 = 0; j0 < n; j0 += kMaxHistJobs) {
        const uint32_t m = std::min<uint32_t>(kMaxHistJobs, n - j0);
        HistJobs jobs{};
        jobs.n = m;
        uint32_t* hp[kMaxHistJobs];
        for (uint32_t k = 0; k < m; k++) hp[k] = d_hists + 768ull * (j0 + k);
        const uint32_t nb = hist_shares(srcs + j0, m, jobs.j, hp);
        CKR_LAUNCH("hist_init_multi_kernel", s, hist_init_multi_kernel<<<m, 256, 0, s>>>(jobs));
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        CKR_LAUNCH("masked_hist_multi_kernel", s, masked_hist_multi_kernel<<<nb, 256, 0, s>>>(jobs));
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

// Small fills used instead of hipMemsetAsync (safe inside captured graphs).
__global__ void set_u64_kernel(uint64_t* p, uint64_t v) { *p = v; }
__global__ void set_u64x_kernel(unsigned long long* p, unsigned long long v) { *p = v; }
hipError_t launch_set_u64(uint64_t* p, uint64_t v, hipStream_t s) {
    CKR_LAUNCH("set_u64_kernel", s, set_u64_kernel<<<1, 1, 0, s>>>(p, v));
    return hipGetLastError();
}
hipError_t launch_set_counter(unsigned long long* p, unsigned long long v, hipStream_t s) {
    CKR_LAUNCH("set_u64x_kernel", s, set_u64x_kernel<<<1, 1, 0, s>>>(p, v));
    return hipGetLastError();
}

// ------------------------------------------------------------------ rANS encode
// Lane state: x, pending output bytes (up to 7, newest lowest) and dword slots
// flushed.  The first byte emitted is the last byte of the lane's stream, so a
// dword taken from the top of the pending bytes, stored little-endian, holds 4
// stream bytes in stream order; slot w (counted from the stream's end) of a
// lane lives at lane_base[w * STRIDE].
struct LaneOut {
    uint32_t x, nacc, w;
    uint64_t acc;
};

__device__ __forceinline__ void lane_init(LaneOut& o) { o.x = L; o.nacc = 0; o.w = 0; o.acc = 0; }

template <uint32_t STRIDE>
__device__ __forceinline__ void push_bytes(LaneOut& o, uint32_t v, uint32_t n, uint32_t* lane_base) {
    o.acc = (o.acc << (8 * n)) | v;
    o.nacc += n;
    if (o.nacc >= 4) {
        lane_base[(uint64_t)o.w * STRIDE] = (uint32_t)(o.acc >> (8 * (o.nacc - 4)));
        o.w++;
        o.nacc -= 4;
    }
}

// One symbol of rans_encode_kernel's loop body (ANSCompressor.cpp:180-202).
// Renormalisation emits at most two bytes (x < 2^32 and xmax >= 2^19); both
// are computed without branches and appended in one step.
template <uint32_t STRIDE>
__device__ __forceinline__ void encode_symbol(LaneOut& o, uint32_t sym, const EncSym* tab, uint32_t* lane_base) {
    const EncSym e = tab[sym];
    if (e.xmax == 0) {  // f == 0: raw byte, no state update (:185-192)
        push_bytes<STRIDE>(o, sym, 1, lane_base);
        return;
    }
    const uint32_t x = o.x;
    const uint32_t e1 = x >= e.xmax ? 1u : 0u;
    const uint32_t x1 = e1 ? (x >> 8) : x;
    const uint32_t e2 = (e1 && x1 >= e.xmax) ? 1u : 0u;
    const uint32_t n = e1 + e2;
    if (n) {
        const uint32_t v = e2 ? (((x & 255u) << 8) | ((x >> 8) & 255u)) : (x & 255u);
        push_bytes<STRIDE>(o, v, n, lane_base);
    }
    const uint32_t xr = e2 ? (x1 >> 8) : x1;
    const uint32_t q = __umulhi(xr, e.rcp) >> (e.cmpl_rsh >> 16);  // q < 2^19 after renormalisation
    o.x = xr + e.bias + __umul24(q, e.cmpl_rsh & 0xFFFFu);
}

template <uint32_t STRIDE>
__device__ __forceinline__ void lane_flush(LaneOut& o, uint32_t* lane_base) {
    if (o.nacc) lane_base[(uint64_t)o.w * STRIDE] = (uint32_t)o.acc;  // low nacc bytes = first stream bytes
}
__device__ __forceinline__ uint32_t lane_bytes(const LaneOut& o) { return o.w * 4 + o.nacc; }

// Canonical streams of the zero planes.  A lane of a masked plane codes K
// zero bytes from state L whatever the data, so its stream depends only on K
// and the table: it is coded once per distinct K (at most three per tensor:
// full units, and the two lane counts of the last unit) instead of once per
// lane, on the host, and stored with launch_canon_store.  Entry i: {K,
// final_state, byte_count, pad} then cw dword slots (the encoder's lane slot
// order); after the three entries, the three streams in byte order.
__device__ __forceinline__ const uint32_t* canon_entry(const uint32_t* canon, uint32_t cw, uint32_t K) {
    // entries hold distinct K values except when two coincide; first match wins
    if (canon[0] == K) return canon;
    if (canon[4 + cw] == K) return canon + 4 + cw;
    return canon + 2 * (4 + cw);
}

template <int SPE>
__device__ __forceinline__ void write_sidecar_row(uint8_t* sidecar, uint64_t pos, uint32_t v, uint32_t nvalid) {
    // pos = tensor byte offset of this 32-bit column (multiple of 4)
    if (SPE == 2) {
        *reinterpret_cast<uint16_t*>(sidecar + (pos >> 1)) = (uint16_t)(v & 0xFFFFu);
    } else if (SPE == 1) {
        const uint64_t e0 = pos >> 1;
        if (nvalid >= 4) *reinterpret_cast<uint16_t*>(sidecar + e0) = (uint16_t)((v & 0xFFu) | ((v >> 8) & 0xFF00u));
        else sidecar[e0] = (uint8_t)(v & 0xFFu);  // one element left (2 valid bytes)
    }
}

template <int SPE>
__device__ __forceinline__ constexpr bool lane_is_live(int b) {
    return SPE == 2 ? (b >= 2) : (SPE == 1 ? (b & 1) == 1 : true);
}

// One wave per unit, one thread per 32-bit column (4 lanes).  Rows are taken
// from the top of the unit down (the reference's reverse order), 8 row loads
// in flight per thread.  DEDUP: lanes of masked planes are not coded; their
// headers come from the canonical streams.
template <int SPE, bool DEDUP>
__global__ void __launch_bounds__(256) encode_kernel(const uint8_t* __restrict__ src, EncodeGeom g, uint64_t u0,
                                                     uint64_t nb, const EncSym* __restrict__ d_enc,
                                                     const uint32_t* __restrict__ canon, uint32_t cw,
                                                     uint32_t* __restrict__ scratch,
                                                     ckr_stream_header* __restrict__ hdrs,
                                                     uint8_t* __restrict__ sidecar,
                                                     const uint32_t* __restrict__ ulist) {
    __shared__ EncSym tab[256];
    tab[threadIdx.x] = d_enc[threadIdx.x];
    __syncthreads();

    const uint32_t j = threadIdx.x & 63;
    const uint64_t ub = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // unit within batch
    if (ub >= nb) return;
    const uint64_t u = ulist ? (uint64_t)ulist[u0 + ub] : u0 + ub;
    const uint64_t ubase = u * g.unit;
    const uint64_t len = (g.n_bytes - ubase < g.unit) ? (g.n_bytes - ubase) : g.unit;
    const uint8_t* usrc = src + ubase;
    uint32_t* uscr = scratch + ub * (uint64_t)g.wmax * 256;
    const uint32_t lm = live_mask32<SPE>();

    LaneOut o[4];
#pragma unroll
    for (int b = 0; b < 4; b++) lane_init(o[b]);

    const uint64_t col = 4ull * j;
    const uint64_t K = (len > col) ? (len - col + 255) / 256 : 0;
    if (K > 0) {
        // top row: may be partial
        const uint64_t k = K - 1;
        const uint64_t p = 256 * k + col;
        const uint32_t nvalid = (uint32_t)((len - p) < 4 ? (len - p) : 4);
        uint32_t v = 0;
        if (nvalid == 4) v = *reinterpret_cast<const uint32_t*>(usrc + p);
        else for (uint32_t b = 0; b < nvalid; b++) v |= (uint32_t)usrc[p + b] << (8 * b);
        if (sidecar && SPE > 0) write_sidecar_row<SPE>(sidecar, ubase + p, v, nvalid);
        v &= lm;
#pragma unroll
        for (int b = 0; b < 4; b++)
            if ((!DEDUP || lane_is_live<SPE>(b)) && (uint32_t)b < nvalid)
                encode_symbol<256>(o[b], (v >> (8 * b)) & 255u, tab, uscr + 4 * j + b);
        // full rows, 8 at a time
        int64_t kk = (int64_t)K - 2;
        for (; kk >= 7; kk -= 8) {
            uint32_t r[8];
#pragma unroll
            for (int i = 0; i < 8; i++) r[i] = *reinterpret_cast<const uint32_t*>(usrc + 256 * (uint64_t)(kk - i) + col);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (sidecar && SPE > 0) write_sidecar_row<SPE>(sidecar, ubase + 256 * (uint64_t)(kk - i) + col, r[i], 4);
                const uint32_t w = r[i] & lm;
#pragma unroll
                for (int b = 0; b < 4; b++)
                    if (!DEDUP || lane_is_live<SPE>(b)) encode_symbol<256>(o[b], (w >> (8 * b)) & 255u, tab, uscr + 4 * j + b);
            }
        }
        for (; kk >= 0; kk--) {
            const uint32_t r = *reinterpret_cast<const uint32_t*>(usrc + 256 * (uint64_t)kk + col);
            if (sidecar && SPE > 0) write_sidecar_row<SPE>(sidecar, ubase + 256 * (uint64_t)kk + col, r, 4);
            const uint32_t w = r & lm;
#pragma unroll
            for (int b = 0; b < 4; b++)
                if (!DEDUP || lane_is_live<SPE>(b)) encode_symbol<256>(o[b], (w >> (8 * b)) & 255u, tab, uscr + 4 * j + b);
        }
    }
    // flush pending bytes and write headers (buf_offset is set by the finalize kernel)
    ckr_stream_header* uh = hdrs + u * 256;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        ckr_stream_header h;
        h.buf_offset = 0;
        h.pad = 0;
        if (DEDUP && !lane_is_live<SPE>(b)) {
            const uint64_t pb = col + b;
            const uint32_t Kb = (uint32_t)(len > pb ? (len - pb + 255) / 256 : 0);
            const uint32_t* ce = canon_entry(canon, cw, Kb);
            h.final_state = ce[1];
            h.byte_count = ce[2];
        } else {
            lane_flush<256>(o[b], uscr + 4 * j + b);
            h.final_state = o[b].x;
            h.byte_count = lane_bytes(o[b]);
        }
        uh[4 * j + b] = h;
    }
}

// Per unit: lane offsets (exclusive scan of byte_count), unit size, and the
// passthrough decision (packed size >= unit length ⇒ raw, ANSCompressor.cpp:694-713).
__global__ void __launch_bounds__(256) unit_finalize_kernel(EncodeGeom g, uint64_t u0,
                                                            ckr_stream_header* __restrict__ hdrs,
                                                            uint32_t* __restrict__ unit_size,
                                                            const uint32_t* __restrict__ ulist) {
    // 64-bit sums: the lanes of a single-unit tensor just below 4 GiB can
    // together exceed 2^32 bytes when the data does not compress (such a unit
    // is then stored raw; the offsets of a coded unit are below its length)
    __shared__ uint64_t sc[256];
    const uint64_t u = ulist ? (uint64_t)ulist[u0 + blockIdx.x] : u0 + blockIdx.x;
    const uint64_t ubase = u * g.unit;
    const uint64_t len = (g.n_bytes - ubase < g.unit) ? (g.n_bytes - ubase) : g.unit;
    const uint32_t t = threadIdx.x;
    ckr_stream_header* uh = hdrs + u * 256;
    const uint32_t c = uh[t].byte_count;
    sc[t] = c;
    __syncthreads();
    for (uint32_t d = 1; d < 256; d <<= 1) {  // inclusive Hillis-Steele scan
        uint64_t v = (t >= d) ? sc[t - d] : 0ull;
        __syncthreads();
        sc[t] += v;
        __syncthreads();
    }
    const uint64_t total = sc[255];
    const bool raw = total >= len;
    if (raw) {
        ckr_stream_header h;
        h.final_state = 0; h.byte_count = (t == 0) ? (uint32_t)len : 0u; h.buf_offset = 0; h.pad = 0;
        uh[t] = h;
    } else {
        uh[t].buf_offset = (uint32_t)(sc[t] - c);
    }
    if (t == 0) unit_size[blockIdx.x] = raw ? (uint32_t)len : (uint32_t)total;
}

// Exclusive scan of unit sizes into unit_off[u0 .. u0+nb] (64-bit), continuing
// from unit_off[u0] written by the previous batch (0 for the first).
__global__ void __launch_bounds__(1024) unit_scan_kernel(const uint32_t* __restrict__ unit_size, uint64_t u0,
                                                         uint64_t nb, uint64_t* __restrict__ unit_off) {
    __shared__ uint64_t sh[1024];
    const uint32_t t = threadIdx.x;
    const uint64_t base = (u0 == 0) ? 0ull : unit_off[u0];  // read before any thread writes
    const uint64_t seg = (nb + 1023) / 1024;
    const uint64_t b0 = t * seg, b1 = (b0 + seg < nb) ? b0 + seg : nb;
    uint64_t s = 0;
    for (uint64_t i = b0; i < b1; i++) s += unit_size[i];
    sh[t] = s;
    __syncthreads();
    for (uint32_t d = 1; d < 1024; d <<= 1) {
        uint64_t v = (t >= d) ? sh[t - d] : 0ull;
        __syncthreads();
        sh[t] += v;
        __syncthreads();
    }
    uint64_t run = base + sh[t] - s;
    for (uint64_t i = b0; i < b1; i++) { unit_off[u0 + i] = run; run += unit_size[i]; }
    if (t == 1023) unit_off[u0 + nb] = base + sh[1023];
}

// Byte sink writing a byte sequence to an arbitrary destination with 32-bit
// stores once the destination is aligned (byte stores only at the ends).
struct ByteSink {
    uint8_t* d;
    uint64_t buf;
    uint32_t nb;
    __device__ __forceinline__ void drain() {
        while (nb > 0 && (reinterpret_cast<uintptr_t>(d) & 3u)) { *d++ = (uint8_t)buf; buf >>= 8; nb--; }
        while (nb >= 4) { *reinterpret_cast<uint32_t*>(d) = (uint32_t)buf; d += 4; buf >>= 32; nb -= 4; }
    }
    __device__ __forceinline__ void push(uint32_t v, uint32_t n) {
        buf |= (uint64_t)v << (8 * nb);
        nb += n;
        drain();
    }
    __device__ __forceinline__ void finish() {
        while (nb > 0) { *d++ = (uint8_t)buf; buf >>= 8; nb--; }
    }
};

// Push one lane stream (slot format: partial dword of r bytes at slot W, then
// slots W-1 .. 0) into the sink; slot loads are issued 16 at a time.
__device__ __forceinline__ void sink_stream(ByteSink& s, const uint32_t* base, uint32_t stride, uint32_t B) {
    const uint32_t W = B >> 2, r = B & 3;
    if (r) s.push(base[(uint64_t)W * stride] & ((1u << (8 * r)) - 1u), r);
    uint32_t w = W;
    for (; w >= 16; w -= 16) {
        uint32_t v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) v[k] = base[(uint64_t)(w - 1 - k) * stride];
#pragma unroll
        for (int k = 0; k < 16; k++) s.push(v[k], 4);
    }
    while (w-- > 0) s.push(base[(uint64_t)w * stride], 4);
}

// Pack every lane stream of a unit to its place, or the masked bytes of a raw
// unit.  One wave per unit; thread j writes the contiguous bytes of lanes
// 4j..4j+3 (zero-plane lanes from the canonical streams when DEDUP).
template <int SPE, bool DEDUP>
__global__ void __launch_bounds__(256) compact_kernel(const uint8_t* __restrict__ src, EncodeGeom g, uint64_t u0,
                                                      uint64_t nb, const uint32_t* __restrict__ scratch,
                                                      const uint32_t* __restrict__ canon, uint32_t cw,
                                                      const ckr_stream_header* __restrict__ hdrs,
                                                      const uint32_t* __restrict__ unit_size,
                                                      const uint64_t* __restrict__ unit_off,
                                                      uint8_t* __restrict__ out,
                                                      const uint32_t* __restrict__ ulist) {
    const uint32_t j = threadIdx.x & 63;
    const uint64_t ub = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (ub >= nb) return;
    const uint64_t u = ulist ? (uint64_t)ulist[u0 + ub] : u0 + ub;
    const uint64_t ubase = u * g.unit;
    const uint64_t len = (g.n_bytes - ubase < g.unit) ? (g.n_bytes - ubase) : g.unit;
    uint8_t* dst = out + unit_off[u];
    const ckr_stream_header* uh = hdrs + u * 256;
    if ((uint64_t)unit_size[ub] == len && uh[0].byte_count == (uint32_t)len && uh[0].final_state == 0) {
        // raw unit: masked bytes, 256 B per row
        for (uint64_t p = 4ull * j; p < len; p += 256) {
            const uint32_t nvalid = (uint32_t)((len - p) < 4 ? (len - p) : 4);
            for (uint32_t b = 0; b < nvalid; b++) {
                const uint8_t v = src[ubase + p + b];
                dst[p + b] = byte_live(p + b, g.es, g.spe) ? v : 0;
            }
        }
        return;
    }
    const uint32_t* uscr = scratch + ub * (uint64_t)g.wmax * 256;
    ByteSink s;
    s.d = dst + uh[4 * j].buf_offset;
    s.buf = 0;
    s.nb = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const uint32_t B = uh[4 * j + b].byte_count;
        if (DEDUP && !lane_is_live<SPE>(b)) {
            const uint64_t pb = 4ull * j + b;
            const uint32_t Kb = (uint32_t)(len > pb ? (len - pb + 255) / 256 : 0);
            sink_stream(s, canon_entry(canon, cw, Kb) + 4, 1, B);
        } else {
            sink_stream(s, uscr + 4 * j + b, 256, B);
        }
    }
    s.finish();
}

__global__ void __launch_bounds__(256) canon_store_kernel(CanonArg a, uint32_t* __restrict__ canon) {
    for (uint32_t i = threadIdx.x; i < a.n; i += blockDim.x) canon[a.off + i] = a.w[i];
}

hipError_t launch_canon_store(const CanonArg& a, uint32_t* canon, hipStream_t s) {
    if (a.n > CANON_ARG_DWORDS) return hipErrorInvalidValue;
    CKR_LAUNCH("canon_store_kernel", s, canon_store_kernel<<<1, 256, 0, s>>>(a, canon));
    return hipGetLastError();
}

template <int SPE, bool DEDUP>
static hipError_t encode_batch_t(const uint8_t* src, const EncodeGeom& g, uint64_t u0, uint64_t nb,
                                 const EncSym* d_enc, const uint32_t* canon, uint32_t cw, uint32_t* scratch,
                                 ckr_stream_header* hdrs, uint8_t* sidecar, uint32_t* unit_size, uint64_t* unit_off,
                                 uint8_t* out, const uint32_t* ulist, hipStream_t s) {
    const uint32_t grid = (uint32_t)((nb + 3) / 4);
    CKR_LAUNCH("encode_kernel", s, encode_kernel<SPE, DEDUP><<<grid, 256, 0, s>>>(src, g, u0, nb, d_enc, canon, cw, scratch, hdrs, sidecar, ulist));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    CKR_LAUNCH("unit_finalize_kernel", s, unit_finalize_kernel<<<(uint32_t)nb, 256, 0, s>>>(g, u0, hdrs, unit_size, ulist));
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (!ulist) {  // a redo batch keeps the offsets the fast kernel published
        CKR_LAUNCH("unit_scan_kernel", s, unit_scan_kernel<<<1, 1024, 0, s>>>(unit_size, u0, nb, unit_off));
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    CKR_LAUNCH("compact_kernel", s, compact_kernel<SPE, DEDUP><<<grid, 256, 0, s>>>(src, g, u0, nb, scratch, canon, cw, hdrs, unit_size, unit_off, out, ulist));
    return hipGetLastError();
}

hipError_t launch_encode_batch(const uint8_t* src, const EncodeGeom& g, uint64_t u0, uint64_t nb, const EncSym* d_enc,
                               const uint32_t* canon, uint32_t cw, bool dedup, uint32_t* scratch,
                               ckr_stream_header* hdrs, uint8_t* sidecar, uint32_t* unit_size, uint64_t* unit_off,
                               uint8_t* out, const uint32_t* ulist, hipStream_t s) {
    if (g.spe == 2)
        return dedup ? encode_batch_t<2, true>(src, g, u0, nb, d_enc, canon, cw, scratch, hdrs, sidecar, unit_size, unit_off, out, ulist, s)
                     : encode_batch_t<2, false>(src, g, u0, nb, d_enc, canon, cw, scratch, hdrs, sidecar, unit_size, unit_off, out, ulist, s);
    if (g.spe == 1)
        return dedup ? encode_batch_t<1, true>(src, g, u0, nb, d_enc, canon, cw, scratch, hdrs, sidecar, unit_size, unit_off, out, ulist, s)
                     : encode_batch_t<1, false>(src, g, u0, nb, d_enc, canon, cw, scratch, hdrs, sidecar, unit_size, unit_off, out, ulist, s);
    return encode_batch_t<0, false>(src, g, u0, nb, d_enc, canon, cw, scratch, hdrs, nullptr, unit_size, unit_off, out, ulist, s);
}

// ------------------------------------------------------------------ fast encode (LDS-staged, look-back)
// Units of at most 64 KiB of masked dtypes, taken in order from a ticket
// counter; one thread per 32-bit column, coding only the two live lanes of its
// column (one coder wave per live plane).  Each live lane writes its stream backward into its
// own LDS slot, so that the stream ends up contiguous and in stream order; the
// slot stride is chosen so that the 64 threads writing their e-th bytes hit
// different banks.  The zero-plane lanes are the canonical streams.  When the
// unit is coded its size is known, its place in the packed output comes from a
// decoupled look-back over the units before it, and the packed bytes are
// written in 16-byte chunks (one wave instruction covers 1 KiB of output).
// A lane that outgrows its slot keeps counting (sizes, states and headers stay
// exact) and the unit's bytes are produced afterwards by the general kernels
// (redo list).
static constexpr uint64_t LB_AGG = 1ull << 62, LB_PFX = 2ull << 62, LB_VAL = (1ull << 62) - 1;
static constexpr uint32_t LB_SPIN_LIMIT = 1u << 20;

struct FastEncParams {
    uint32_t sl0, sl1;          // LDS slot bytes per lane, live lanes of rank 0 and 1 (multiples of 4)
    uint32_t stride0, stride1;  // slot strides (slot bytes + bank padding)
    uint32_t cw;                // canonical entry size (dwords after the 4 header words)
    uint32_t canon_bytes;       // bytes per canonical entry in the LDS copy (stream order)
};

// Encode table entry in LDS, 16 bytes, every field ready for its instruction
// (one ds_read_b128 per symbol): x = rcp; y = cmpl | rsh << 24 (the 24-bit
// multiply reads cmpl, the shift reads byte 3); z = bias; w = 8f (the
// renormalisation compares read it against bytes of the state).  See EncSym:
// cmpl = M - f, rsh < 12, bias < 8192; w = 0 marks f == 0.
__device__ __forceinline__ uint4 enc_quad(const EncSym& e) {
    return make_uint4(e.rcp, (e.cmpl_rsh & 0xFFFu) | ((e.cmpl_rsh >> 16) << 24), e.bias, e.xmax >> 16);
}

// Lane coder state.  x: rANS state.  {hi, lo}: the last 8 bytes emitted, the
// newest in the top byte of hi.  sel: v_perm selector 0x08090A0B - P*0x01010101
// with P (0..7) the emitted bytes not yet flushed (the top P bytes of the
// window).  ptr: LDS byte address of the lane's next flushed dword.
struct EncLane {
    uint32_t x, hi, lo, sel, ptr;
};

// One symbol of rans_encode_kernel's loop body (ANSCompressor.cpp:180-202)
// without branches, from the table entry t (see enc_quad).  Renormalisation
// emits n in {0,1,2} bytes: x >= f*2^19 and x >= f*2^27 are (x >> 16) >= 8f
// and (x >> 24) >= 8f.  The n low bytes of x, low byte first (the reference's
// emission order), enter the window from the top: one v_alignbyte per register
// shifts by n bytes.  ESC: the table may give f == 0 to a symbol of the data
// (raw-byte escape, no state update, :185-192); tables built from the data
// itself never do.
template <bool ESC>
__device__ __forceinline__ void enc_step(EncLane& s, uint32_t sym, uint4 t) {
    const uint32_t f8 = t.w;
    const uint32_t x = s.x;
    uint32_t n4 = ((x >> 24) >= f8) ? 0x02020202u : (((x >> 16) >= f8) ? 0x01010101u : 0u);
    uint32_t ins = x;
    bool esc = false;
    if (ESC) {
        esc = f8 == 0u;
        n4 = esc ? 0x01010101u : n4;
        ins = esc ? sym : x;
    }
    const uint32_t xr = __builtin_amdgcn_alignbyte(0u, x, n4);
    s.lo = __builtin_amdgcn_alignbyte(s.hi, s.lo, n4);
    s.hi = __builtin_amdgcn_alignbyte(ins, s.hi, n4);
    s.sel -= n4;
    const uint32_t q = __umulhi(xr, t.x) >> (t.y >> 24);
    const uint32_t xn = xr + t.z + __umul24(q, t.y);
    s.x = (ESC && esc) ? x : xn;
}

// Flush the 4 oldest pending bytes when P >= 4 (called at least every 2
// symbols, so P <= 7).  The dword holds them in stream order (the newest at the
// lowest address): a byte-reversing select out of the 8-byte window.
// The dword is stored whatever P: with P < 4 it lands at the lane's next
// flush position, which a later flush or the final partial dword overwrites,
// or, when the stream ends on a dword boundary, just below the stream (in the
// slot, its padding or the guard).  P >= 4 exactly when bit 3 of the
// selector's low byte (0x0B - P) is clear.
__device__ __forceinline__ void enc_flush(EncLane& s, uint8_t* lds8) {
    *reinterpret_cast<uint32_t*>(lds8 + s.ptr) = __builtin_amdgcn_perm(s.hi, s.lo, s.sel);
    const bool fl = (s.sel & 8u) == 0u;
    s.ptr -= fl ? 4u : 0u;
    s.sel += fl ? 0x04040404u : 0u;
}

// End of the lane: the remaining P (< 4 after a flush) bytes go into the top of
// one more dword (its lower bytes lie before the stream's start).  Returns the
// byte count; the stream then occupies [slot_end - count, slot_end).
__device__ __forceinline__ uint32_t enc_finish(EncLane& s, uint8_t* lds8, uint32_t slot_end) {
    enc_flush(s, lds8);
    const uint32_t P = 0x0Bu - (s.sel & 0xFFu);
    *reinterpret_cast<uint32_t*>(lds8 + s.ptr) = __builtin_amdgcn_perm(s.hi, s.lo, s.sel);
    return (slot_end - 4u - s.ptr) + P;
}

// Look-back status words.  Their values carry everything the protocol needs
// (sizes and prefixes); no other data is published through them, so relaxed
// device-scope atomics suffice — acquire/release at this scope would write
// back or invalidate the whole L2 of the XCD on every access.
__device__ __forceinline__ uint64_t lb_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void lb_store(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void lb_max(uint64_t* p, uint64_t v) {
    (void)__hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exclusive prefix of the packed sizes of units [0, u), computed by the whole
// wave, in two levels.  Unit words status[v] hold v's size (AGG) and then its
// inclusive prefix (PFX).  Units form blocks of 64; block words bs[c] (after the
// n unit words) hold the block's size once all of its units have published
// theirs (the last one to add itself to the block's count in bacc[c], which
// packs count << 40 | sum, publishes it) and then the inclusive prefix through
// the block (published by the block's last unit).  Block words only ever grow
// (atomic max; PFX > AGG), so a late AGG cannot overwrite a PFX.  The walk
// reads the units of u's own block before u (one step of 64 lanes) and then
// whole blocks, 64 per step, back to the nearest prefix, so that a unit whose
// nearest published prefix lies hundreds of units back still needs about two
// round trips.  Every unit before u holds a ticket taken earlier, so it is
// running or done and will publish; the wait is bounded all the same (error
// flag, no hang).
__device__ uint64_t lookback_wave(uint64_t* status, uint64_t n_units, uint64_t u, uint64_t size, uint32_t* err,
                                  uint32_t j) {
    const uint64_t nblk = (n_units + 63) >> 6;
    uint64_t* bs = status + n_units;
    uint64_t* bacc = bs + nblk;
    const uint64_t b = u >> 6, u0 = b << 6;
    if (j == 0) {
        lb_store(&status[u], (u == 0 ? LB_PFX : LB_AGG) | size);
        const uint64_t old = __hip_atomic_fetch_add(&bacc[b], (1ull << 40) | size, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t in_blk = (n_units - u0 < 64) ? n_units - u0 : 64;
        if ((old >> 40) + 1 == in_blk) lb_max(&bs[b], LB_AGG | ((old & ((1ull << 40) - 1)) + size));
    }
    uint64_t excl = 0;
    bool done = u == 0;
    uint32_t spins = 0;
    const uint32_t na = (uint32_t)(u - u0);  // units of u's block before u
    while (!done && na > 0) {
        const bool act = j < na;
        const uint64_t st = act ? lb_load(&status[u - 1 - j]) : 0ull;
        const uint64_t pfx = __ballot(act && (st >> 62) == 2);
        const uint32_t stop = pfx ? (uint32_t)__builtin_ctzll(pfx) : 64u;  // nearest prefix
        const bool need = act && j <= stop;
        if (__ballot(need && (st >> 62) == 0)) {  // a unit not published yet
            if (++spins > LB_SPIN_LIMIT) { if (j == 0) atomicOr(err, 1u); done = true; break; }
            __builtin_amdgcn_s_sleep(2);
            continue;
        }
        uint64_t v = need ? (st & LB_VAL) : 0ull;
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
        excl += v;
        done = pfx != 0;
        break;
    }
    int64_t bb = (int64_t)b;  // blocks < bb remain
    while (!done && bb > 0) {
        const int64_t idx = bb - 1 - (int64_t)j;
        const uint64_t st = idx >= 0 ? lb_load(&bs[idx]) : LB_PFX;
        const uint64_t pfx = __ballot((st >> 62) == 2);
        const uint32_t stop = pfx ? (uint32_t)__builtin_ctzll(pfx) : 63u;  // last lane needed
        const uint64_t need = (stop == 63u) ? ~0ull : ((2ull << stop) - 1);
        if (__ballot((st >> 62) == 0) & need) {  // a block not complete yet
            if (++spins > LB_SPIN_LIMIT) { if (j == 0) atomicOr(err, 1u); break; }
            __builtin_amdgcn_s_sleep(2);
            continue;
        }
        uint64_t v = (j <= stop) ? (st & LB_VAL) : 0ull;
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
        excl += v;
        if (pfx) break;
        bb -= 64;
    }
    if (j == 0) {
        if (u > 0) lb_store(&status[u], LB_PFX | (excl + size));
        if (u == u0 + 63 || u + 1 == n_units) lb_max(&bs[b], LB_PFX | (excl + size));
    }
    return excl;
}

// 16 LDS bytes from an arbitrary byte address (5 aligned 32-bit reads).
__device__ __forceinline__ uint4 lds_read16(const uint8_t* lds8, uint32_t a) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(lds8 + (a & ~3u));
    const uint32_t sh = a & 3u;
    const uint32_t d0 = w[0], d1 = w[1], d2 = w[2], d3 = w[3], d4 = w[4];
    return make_uint4(__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh),
                      __builtin_amdgcn_alignbyte(d3, d2, sh), __builtin_amdgcn_alignbyte(d4, d3, sh));
}

// Bytes [s, 16) of r over those of v (0 <= s < 16): one bitfield insert per
// dword, the mask of dword d being the bytes at or above s - 4d.
__device__ __forceinline__ uint4 merge16_from(uint4 v, uint4 r, uint32_t s) {
    auto m = [&](int d) {
        const int32_t k = min(max((int32_t)s - 4 * d, 0), 4);  // bytes kept from v
        return k >= 4 ? 0u : (0xFFFFFFFFu << (8 * k));
    };
    return make_uint4((r.x & m(0)) | (v.x & ~m(0)), (r.y & m(1)) | (v.y & ~m(1)), (r.z & m(2)) | (v.z & ~m(2)),
                      (r.w & m(3)) | (v.w & ~m(3)));
}


// Coding of the live lanes of every column of a unit whose rows are all full
// (length a multiple of 256, so every column has the same nrows rows).  P = 0:
// byte FL of each column (chain c0); P = 1: byte 3 (chain c0); P = 2: both
// (c0: byte FL, c1: byte 3, interleaved).  Rows are taken from the top down.
// The rows above the highest multiple of GR go one at a time; then groups of
// GR rows, the next group's loads in flight while the current one is coded
// (loads and table reads are unconditional, so the waits stay exact), and each
// TB-row batch's table entries read while the batch before it is coded.
// Pending bytes are flushed after every second row.  The sidecar rows are
// written by the thread coding plane 0 and 1 alternately (row k by P == k & 1),
// or all of them when P = 2.
template <int SPE, bool ESC, bool SIDE, int P, int GR, int TB, int NBUF>
__device__ __forceinline__ void enc_full_rows(EncLane& c0, EncLane& c1, const uint8_t* ucol, uint8_t* sidecar,
                                              uint64_t ubase, uint32_t j, uint32_t nrows, const uint4* tab,
                                              uint8_t* lds8) {
    constexpr int FL = SPE == 2 ? 2 : 1;
    constexpr uint32_t SH0 = P == 1 ? 24u : 8u * FL;  // byte of chain c0
    constexpr uint32_t SH1 = 24u;                     // byte of chain c1 (P = 2)
    const uint32_t* in32 = reinterpret_cast<const uint32_t*>(ucol);          // row k at in32[64 k]
    uint16_t* sc16 = SIDE ? reinterpret_cast<uint16_t*>(sidecar + (ubase >> 1) + 2 * j) : nullptr;  // row k at sc16[64 k]
    auto side = [&](uint16_t* p, uint32_t wd) {
        if (SIDE) *p = (uint16_t)(SPE == 2 ? (wd & 0xFFFFu) : ((wd & 0xFFu) | ((wd >> 8) & 0xFF00u)));
    };
    auto mine = [&](uint32_t k) { return P == 2 || (k & 1u) == (uint32_t)P; };  // sidecar row k written here
    static_assert(GR % TB == 0 && TB % 2 == 0 && GR % 2 == 0, "row groups of whole table batches");
    const uint32_t ng = nrows / GR;  // full groups: rows [0, GR ng)
    for (int32_t k = (int32_t)nrows - 1; k >= (int32_t)(GR * ng); k--) {
        const uint32_t wd = in32[64 * k];
        if (mine((uint32_t)k)) side(sc16 + 64 * k, wd);
        const uint32_t s0 = (wd >> SH0) & 255u;
        enc_step<ESC>(c0, s0, tab[s0]);
        if (P == 2) { const uint32_t s1 = wd >> SH1; enc_step<ESC>(c1, s1, tab[s1]); }
        if ((k & 1) == 0) { enc_flush(c0, lds8); if (P == 2) enc_flush(c1, lds8); }
    }
    enc_flush(c0, lds8);
    if (P == 2) enc_flush(c1, lds8);
    if (ng == 0) return;
    // group g: rows GR g + GR - 1 (r[0]) down to GR g (r[GR - 1])
    auto load = [&](uint32_t (&r)[GR], uint32_t g) {
        const uint32_t* p = in32 + 64 * (GR * g + GR - 1);
#pragma unroll
        for (int i = 0; i < GR; i++) r[i] = p[-64 * i];
    };
    auto code = [&](const uint32_t (&r)[GR], uint32_t g) {
        uint4 t0[2][TB], t1[2][TB];
        (void)t1;
        auto fetch = [&](int buf, int i0) {
#pragma unroll
            for (int i = 0; i < TB; i++) {
                t0[buf][i] = tab[(r[i0 + i] >> SH0) & 255u];
                if (P == 2) t1[buf][i] = tab[r[i0 + i] >> SH1];
            }
        };
        uint16_t* scp = SIDE ? sc16 + 64 * (GR * g + GR - 1) : nullptr;
        constexpr int NB = GR / TB;
        fetch(0, 0);
#pragma unroll
        for (int bt = 0; bt < NB; bt++) {
            if (bt < NB - 1) fetch((bt + 1) & 1, TB * (bt + 1));
#pragma unroll
            for (int i = 0; i < TB; i++) {
                const int ii = TB * bt + i;              // row GR g + GR - 1 - ii: parity (ii & 1) ^ 1
                if (P == 2 || ((ii & 1) ^ 1) == P) side(scp - 64 * ii, r[ii]);
                enc_step<ESC>(c0, (r[ii] >> SH0) & 255u, t0[bt & 1][i]);
                if (P == 2) enc_step<ESC>(c1, r[ii] >> SH1, t1[bt & 1][i]);
                if (i & 1) { enc_flush(c0, lds8); if (P == 2) enc_flush(c1, lds8); }
            }
        }
    };
    if (NBUF == 2) {
        uint32_t ra[GR], rb[GR];
        uint32_t g = ng - 1;
        load(ra, g);
        for (;;) {
            if (g == 0) { code(ra, 0); break; }
            load(rb, g - 1);
            code(ra, g);
            g--;
            if (g == 0) { code(rb, 0); break; }
            load(ra, g - 1);
            code(rb, g);
            g--;
        }
    } else {
        // three buffers: group g - 2's loads issued while group g is coded (the
        // last groups load group 0 again, so that every load is unconditional)
        uint32_t ra[GR], rb[GR], rc[GR];
        int32_t g = (int32_t)ng - 1;
        load(ra, (uint32_t)g);
        load(rb, (uint32_t)max(g - 1, 0));
        for (;;) {
            load(rc, (uint32_t)max(g - 2, 0));
            code(ra, (uint32_t)g);
            if (g == 0) break;
            g--;
            load(ra, (uint32_t)max(g - 2, 0));
            code(rb, (uint32_t)g);
            if (g == 0) break;
            g--;
            load(rb, (uint32_t)max(g - 2, 0));
            code(rc, (uint32_t)g);
            if (g == 0) break;
            g--;
        }
    }
}

// Warp-specialised persistent workgroups, one per CU: WS pairs of (2 coder
// waves, NPK packer waves), each pair with two LDS slot sets used in turn.  The
// coder waves of a pair (byte FL and byte 3 of every column) take a unit from
// the ticket counter, code it into the free set and hand it over; the packer
// waves compute its lane sizes, publish its size, run the look-back (one
// wave), write its headers and lane records (another), pack its bytes (all of
// them), and give the set back.  Coding therefore never
// waits for the look-back; it waits only while both sets of its pair are in
// the packers' hands.  Hand-overs are workgroup-scope LDS counters (a release
// fence, then one lane's atomic add, on the producer side; acquire polls with
// s_sleep on the consumer side).
//
// LDS layout (bytes): table 256 x 16 (see enc_quad) | canonical headers 12 x
// u32 | canonical bytes 3 x canon_bytes | pair control blocks | 2 x WS regions
// | 32 bytes of read padding.  A region holds one set: the packers' lane
// records (per lane {LDS address of unit byte 0 as if it were in the lane, end
// of the lane in the unit}, 8 bytes) and block map (u8 lane per 64 bytes of
// packed output), then the rank-0 slots (64 x stride0) and the rank-1 slots
// (64 x stride1).  The records and the map are only written once both coders
// are done with the set, so they
// double as the guard under the slots: a lane's dwords are flushed downward
// from the end of its slot, and a lane that outgrows its slot keeps flushing
// into the slots below it (lanes of the same unit, whose bytes are then redone
// by the general kernels) and, for the lowest slot, into the lane tables (at
// most 2 bytes per symbol, 256 symbols: 516 bytes), never out of its region.
static constexpr uint32_t FE_TABSZ = 4096, FE_CHDR = FE_TABSZ, FE_CBYTES = FE_TABSZ + 48;
// Rows per load group and per table batch of the fast encoder's coders.
static constexpr int ENC_GR = 32, ENC_TB = 2, ENC_NBUF = 2;
// Packer waves per coder pair.  With four, a workgroup of two pairs is 12
// waves (3 per SIMD); the coders are held to 128 VGPRs (4 waves per SIMD) so
// that the overlapped histogram's wave still fits on every SIMD beside them.
static constexpr int ENC_NPK = 4;
static constexpr uint32_t R_REC = 0, R_MAP = 2048, R_SLOTS = 3076;
static_assert(R_SLOTS >= 516 && R_SLOTS % 4 == 0 && R_MAP >= R_REC + 256 * 8 && R_SLOTS >= R_MAP + 1025,
              "region: lane records, block map and guard under the slots");

struct WsPairCtl {
    uint32_t unit[2];         // unit in set s (>= n_units: none left, the pair stops)
    uint32_t coded[2];        // +1 by each coder wave per use of set s
    uint32_t freed[2];        // +1 by the packers per use of set s
    uint32_t tick;            // uses started by the plane-FL coder (unit published)
    uint32_t pbar;            // barrier count of the packer waves
    uint32_t off[2][2];       // packed offset of the unit in set s (lo, hi)
    uint32_t xread;           // +1 by each packer wave per use, once it holds the exchange words
    uint32_t pad[3];
};
static_assert(sizeof(WsPairCtl) % 16 == 0, "control block alignment");

__device__ __forceinline__ uint32_t ws_load(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void ws_wait_ge(const uint32_t* p, uint32_t v) {
    while (ws_load(p) < v) __builtin_amdgcn_s_sleep(1);
}
// Makes the wave's earlier LDS (and global) writes visible in the workgroup,
// then adds v to *p once for the wave.
__device__ __forceinline__ void ws_signal(uint32_t* p, uint32_t v, uint32_t lane) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) (void)__hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// 4 bytes between slots: a stream that fills its slot exactly still writes one
// dword below its start (the final partial dword, empty)
__host__ __device__ constexpr uint32_t slot_stride(uint32_t sl) { return sl + 4; }
__host__ __device__ constexpr uint32_t ws_ctl_offset(uint32_t canon_bytes) {
    return (FE_CBYTES + 3 * canon_bytes + 15u) & ~15u;
}
__host__ __device__ constexpr uint32_t ws_region_bytes(uint32_t stride0, uint32_t stride1) {
    return (R_SLOTS + 64 * stride0 + 64 * stride1 + 15u) & ~15u;
}
__host__ __device__ constexpr uint32_t ws_lds_bytes(uint32_t pairs, uint32_t canon_bytes, uint32_t stride0,
                                                    uint32_t stride1) {
    return ws_ctl_offset(canon_bytes) + pairs * (uint32_t)sizeof(WsPairCtl) +
           2 * pairs * ws_region_bytes(stride0, stride1) + 32;
}

// LIST: the units a previous launch put on the redo list (ctl[1] of them in
// redo_list) coded again with slots large enough for any lane (2 bytes per
// row), at the offsets that launch published; tickets from ctl[3]; no sidecar,
// no look-back.  A lane that outgrew even those slots would set ctl[2] bit 1.
template <int SPE, bool ESC, bool SIDE, int PAIRS, int NPK, bool LIST>
__device__ __forceinline__ void encode_fast_body(const uint8_t* __restrict__ src, EncodeGeom g,
                                                 const EncSym* __restrict__ d_enc,
                                                 const uint32_t* __restrict__ canon, FastEncParams fp,
                                                 ckr_stream_header* __restrict__ hdrs,
                                                 uint8_t* __restrict__ sidecar, uint8_t* __restrict__ out,
                                                 uint64_t* __restrict__ unit_off,
                                                 uint64_t* __restrict__ status, uint32_t* __restrict__ ctl,
                                                 uint32_t* __restrict__ redo_list,
                                                 uint64_t* __restrict__ phase,
                                                 const uint32_t* __restrict__ dsl) {
    if (LIST && __hip_atomic_load(&ctl[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) return;  // nothing to redo
    if (dsl) {  // slot sizes made on the device (table_enc_kernel), within the launch's LDS
        fp.sl0 = dsl[0]; fp.sl1 = dsl[1];
        fp.stride0 = slot_stride(fp.sl0); fp.stride1 = slot_stride(fp.sl1);
    }
    extern __shared__ uint32_t lds[];
    uint8_t* lds8 = reinterpret_cast<uint8_t*>(lds);
    constexpr uint32_t NT = 64 * (2 + NPK) * PAIRS;
    const uint4* tab = reinterpret_cast<const uint4*>(lds8 + 0);
    uint32_t* chdr = reinterpret_cast<uint32_t*>(lds8 + FE_CHDR);
    const uint32_t cb_off = FE_CBYTES;
    const uint32_t ctl_off = ws_ctl_offset(fp.canon_bytes);
    const uint32_t rbytes = ws_region_bytes(fp.stride0, fp.stride1);
    const uint32_t reg0 = ctl_off + PAIRS * (uint32_t)sizeof(WsPairCtl);
    const uint32_t tid = threadIdx.x;
    const uint32_t j = tid & 63;  // column
    constexpr int FL = SPE == 2 ? 2 : 1;  // byte of the first live lane in a column
    const uint32_t lm = live_mask32<SPE>();

    {   // table (EncSym → enc_quad), canonical headers and canonical streams (byte order), control blocks
        const uint4* d_tab = reinterpret_cast<const uint4*>(d_enc);
        uint4* wt = reinterpret_cast<uint4*>(lds8 + 0);
        for (uint32_t k = tid; k < 256; k += NT) {
            const uint4 tv = d_tab[k];
            const EncSym e = {tv.x, tv.y, tv.z, tv.w};
            wt[k] = enc_quad(e);
        }
        const uint32_t* cs = canon + 3 * (4 + fp.cw);
        uint32_t* cb32 = reinterpret_cast<uint32_t*>(lds8 + cb_off);
        const uint32_t ncb = 3 * fp.canon_bytes / 4;
        const uint32_t cb_per = fp.canon_bytes / 4;
        for (uint32_t i = tid; i < ncb; i += NT) cb32[i] = cs[(i / cb_per) * fp.cw + (i % cb_per)];
        if (tid < 12) chdr[tid] = canon[(tid >> 2) * (4 + fp.cw) + (tid & 3)];
        uint32_t* c32 = reinterpret_cast<uint32_t*>(lds8 + ctl_off);
        for (uint32_t i = tid; i < PAIRS * (uint32_t)sizeof(WsPairCtl) / 4; i += NT) c32[i] = 0;
    }
    __syncthreads();

    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    // waves 0 .. 2 PAIRS - 1 code, the others pack, NPK per pair (wave w runs on
    // SIMD w mod 4, so the coders are on four different SIMDs)
    const bool coder = wv < 2 * PAIRS;
    const uint32_t pr = coder ? (wv >> 1) : (wv - 2 * PAIRS) / NPK;  // pair
    const uint32_t rl = wv & 1;  // coder: 0 byte FL, 1 byte 3
    const uint32_t pw = coder ? 0u : (wv - 2 * PAIRS) % NPK;  // packer: 0 look-back, 1 headers, all pack
    WsPairCtl& pc = *reinterpret_cast<WsPairCtl*>(lds8 + ctl_off + pr * (uint32_t)sizeof(WsPairCtl));
    const uint32_t col = 4 * j;

    if (coder) {
        const uint32_t sh = rl ? 24u : 8u * FL;  // this wave's byte of the column
        for (uint32_t i = 0;; i++) {
            const uint32_t s = i & 1;
            const uint64_t t_wait = phase ? wall_clock64() : 0;
            if (i >= 2) ws_wait_ge(&pc.freed[s], i >> 1);  // set s given back
            if (rl == 0) {
                if (j == 0) {  // ticket
                    if (LIST) {
                        const uint32_t t = atomicAdd(&ctl[3], 1u);
                        pc.unit[s] = t < ctl[1] ? redo_list[t] : (uint32_t)g.n_units;
                    } else {
                        pc.unit[s] = atomicAdd(&ctl[0], 1u);
                    }
                }
                ws_signal(&pc.tick, 1u, j);
            } else {
                ws_wait_ge(&pc.tick, i + 1);
            }
            const uint32_t u = __builtin_amdgcn_readfirstlane(ws_load(&pc.unit[s]));
            if (u >= g.n_units) {
                ws_signal(&pc.coded[s], 1u, j);
                break;
            }
            const uint64_t t_start = phase ? wall_clock64() : 0;
            const uint64_t ubase = (uint64_t)u * g.unit;
            const uint32_t len = (uint32_t)((g.n_bytes - ubase < g.unit) ? (g.n_bytes - ubase) : g.unit);
            const uint8_t* usrc = src + ubase;
            const uint32_t rb = reg0 + (2 * pr + s) * rbytes;
            const uint32_t endw = rl ? rb + R_SLOTS + 64 * fp.stride0 + j * fp.stride1 + fp.sl1
                                     : rb + R_SLOTS + j * fp.stride0 + fp.sl0;
            EncLane c{L, 0u, 0u, 0x08090A0Bu, endw - 4u};
            EncLane c_unused = c;
            const uint32_t K = len > col ? (len - col + 255) / 256 : 0u;
            if ((len & 255u) == 0) {
                if (rl == 0) enc_full_rows<SPE, ESC, SIDE, 0, ENC_GR, ENC_TB, ENC_NBUF>(c, c_unused, usrc + col, sidecar, ubase, j, len >> 8, tab, lds8);
                else enc_full_rows<SPE, ESC, SIDE, 1, ENC_GR, ENC_TB, ENC_NBUF>(c, c_unused, usrc + col, sidecar, ubase, j, len >> 8, tab, lds8);
            } else {
                // A tensor's last unit: rows from the top down, one at a time; the top
                // row may be partial (bf16: lane 4j+3 has one symbol fewer).
                for (int32_t k = (int32_t)K - 1; k >= 0; k--) {
                    const uint32_t p = 256 * (uint32_t)k + col;
                    const uint32_t nvalid = (len - p) < 4 ? (len - p) : 4;
                    uint32_t v = 0;
                    if (nvalid == 4) v = *reinterpret_cast<const uint32_t*>(usrc + p);
                    else for (uint32_t b = 0; b < nvalid; b++) v |= (uint32_t)usrc[p + b] << (8 * b);
                    if (SIDE && (uint32_t)(k & 1) == rl) write_sidecar_row<SPE>(sidecar, ubase + p, v, nvalid);
                    v &= lm;
                    const uint32_t sy = (v >> sh) & 255u;
                    if (rl == 0 || nvalid == 4) enc_step<ESC>(c, sy, tab[sy]);
                    if ((k & 1) == 0) enc_flush(c, lds8);
                }
            }
            const uint32_t e = enc_finish(c, lds8, endw);
            // per column: count FL, state FL, count 3, state 3, in the set's lane-record
            // area (the records are written only after every packer wave has read
            // them; it lies below the guard that an outgrown lowest slot may write into)
            uint32_t* xch = reinterpret_cast<uint32_t*>(lds8 + rb + R_REC);
            xch[2 * rl * 64 + j] = e;
            xch[(2 * rl + 1) * 64 + j] = c.x;
            ws_signal(&pc.coded[s], 1u, j);
            if (phase && rl == 0 && j == 0) {
                uint64_t* ph = phase + 8 * (uint64_t)u;
                ph[0] = t_wait; ph[1] = t_start; ph[2] = wall_clock64();
            }
        }
        return;
    }

    // packer waves
    uint32_t bar = 0;
    auto pbar_sync = [&]() {
        bar += NPK;
        ws_signal(&pc.pbar, 1u, j);
        ws_wait_ge(&pc.pbar, bar);
    };
    for (uint32_t i = 0;; i++) {
        const uint32_t s = i & 1;
        ws_wait_ge(&pc.coded[s], 2 * ((i >> 1) + 1));
        const uint32_t u = __builtin_amdgcn_readfirstlane(ws_load(&pc.unit[s]));
        if (u >= g.n_units) break;
        const uint64_t t_seen = phase ? wall_clock64() : 0;
        const uint64_t ubase = (uint64_t)u * g.unit;
        const uint32_t len = (uint32_t)((g.n_bytes - ubase < g.unit) ? (g.n_bytes - ubase) : g.unit);
        const uint8_t* usrc = src + ubase;
        const uint32_t rb = reg0 + (2 * pr + s) * rbytes;
        uint2* lrec = reinterpret_cast<uint2*>(lds8 + rb + R_REC);  // per lane {LDS address of unit byte 0, lane end}
        static_assert(R_REC + 1024 <= R_SLOTS - 516, "exchange words below the guard of the lowest slot");
        uint8_t* bmap_w = lds8 + rb + R_MAP;                           // 64-byte block → lane (1025)
        const uint32_t end0 = rb + R_SLOTS + j * fp.stride0 + fp.sl0;
        const uint32_t end1 = rb + R_SLOTS + 64 * fp.stride0 + j * fp.stride1 + fp.sl1;
        const uint32_t* xch = reinterpret_cast<const uint32_t*>(lds8 + rb + R_REC);
        const uint32_t e0 = xch[j], x0 = xch[64 + j];
        const uint32_t e1 = xch[128 + j], x1 = xch[192 + j];
        ws_signal(&pc.xread, 1u, j);  // once all NPK have, the records may overwrite them
        // byte counts, final states and LDS stream starts of the four lanes of column j
        uint32_t cnt[4], fs[4], sa[4];
#pragma unroll
        for (int b = 0; b < 4; b++) {
            if (b == FL) { cnt[b] = e0; fs[b] = x0; sa[b] = end0 - e0; }
            else if (b == 3) { cnt[b] = e1; fs[b] = x1; sa[b] = end1 - e1; }
            else {
                const uint32_t pb = col + b;
                const uint32_t Kb = len > pb ? (len - pb + 255) / 256 : 0u;
                const uint32_t ent = (chdr[0] == Kb) ? 0u : ((chdr[4] == Kb) ? 1u : 2u);
                fs[b] = chdr[4 * ent + 1];
                cnt[b] = chdr[4 * ent + 2];
                sa[b] = cb_off + ent * fp.canon_bytes;
            }
        }
        const uint32_t tsum = cnt[0] + cnt[1] + cnt[2] + cnt[3];
        uint32_t incl = tsum;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t v = __shfl_up(incl, d, 64);
            if ((int)j >= d) incl += v;
        }
        const uint32_t total = __shfl(incl, 63, 64);
        const uint32_t excl = incl - tsum;
        const bool raw = total >= len;
        const uint32_t size = raw ? len : total;
        // the lowest dword a lane wrote must lie in its slot
        const bool over = ((e0 + 3u) & ~3u) > fp.sl0 || ((e1 + 3u) & ~3u) > fp.sl1;
        const bool any_over = __ballot(over) != 0;

        uint64_t t_off = 0;
        if (pw == 1) {
            // headers (4 per thread, 64 contiguous bytes) and the lane tables for packing
            ckr_stream_header* uh = hdrs + (uint64_t)u * 256 + 4 * j;
            uint32_t run = excl;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                ckr_stream_header h;
                if (raw) {
                    h.final_state = 0; h.byte_count = (j == 0 && b == 0) ? len : 0u; h.buf_offset = 0;
                } else {
                    h.final_state = fs[b]; h.byte_count = cnt[b]; h.buf_offset = run;
                }
                h.pad = 0;
                uh[b] = h;
                run += cnt[b];
            }
            // lane records and the block map (the lane holding the first byte of each
            // 64-byte block of the packed unit), the records written over the exchange
            // words once every packer wave holds them
            ws_wait_ge(&pc.xread, (i + 1) * NPK);
            run = excl;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                lrec[4 * j + b] = make_uint2(sa[b] - run, run + cnt[b]);
                if (!raw)
                    for (uint32_t blk = (run + 63u) >> 6; (blk << 6) < run + cnt[b]; blk++) bmap_w[blk] = (uint8_t)(4 * j + b);
                run += cnt[b];
            }
        } else if (pw == 0 && LIST) {  // the offset published by the first launch
            if (j == 0) {
                const uint64_t off = unit_off[u];
                pc.off[s][0] = (uint32_t)off;
                pc.off[s][1] = (uint32_t)(off >> 32);
            }
        } else if (pw == 0) {
            const uint64_t off = lookback_wave(status, g.n_units, u, size, &ctl[2], j);
            if (j == 0) {
                unit_off[u] = off;
                if (u + 1 == g.n_units) {  // the total, also beside the control words (one read-back)
                    unit_off[u + 1] = off + size;
                    *reinterpret_cast<unsigned long long*>(ctl + 4) = off + size;
                }
                pc.off[s][0] = (uint32_t)off;
                pc.off[s][1] = (uint32_t)(off >> 32);
            }
            t_off = phase ? wall_clock64() : 0;
        }
        pbar_sync();
        uint32_t nchunks = 0;
        const uint64_t off = (uint64_t)pc.off[s][0] | ((uint64_t)pc.off[s][1] << 32);
        uint8_t* dst = out + off;
        if (raw) {  // masked bytes of the unit, byte stores (rare)
            for (uint32_t q = 64 * pw + j; q < len; q += 64 * NPK) {
                const uint8_t v = usrc[q];
                dst[q] = byte_live(q, g.es, g.spe) ? v : 0;
            }
        } else if (any_over) {  // bytes come from a redo launch
            if (pw == 0 && j == 0) {
                if (LIST) atomicOr(&ctl[2], 2u);  // (never: these slots hold 2 bytes per row)
                else redo_list[atomicAdd(&ctl[1], 1u)] = u;
            }
        } else {
            // Packed bytes in 16-byte destination chunks aligned in global memory,
            // 64 consecutive chunks (1 KiB of output, whole cache lines) per wave
            // store: the NPK packer waves take rounds of 64 chunks in turn.  Chunk
            // c starts at unit byte q = qbase + 16c (chunk 0 may start up to 15
            // bytes before the unit).  Its first lane: the block map gives the lane
            // holding the first byte of the chunk's 64-byte block, and the lanes
            // after it are stepped over while they end at or before the chunk's
            // first byte; the bytes past that lane's end come from the following
            // non-empty lanes.  Bytes outside the unit (its first and last chunks
            // are shared with the neighbouring units) are not stored.
            const uint64_t ab = reinterpret_cast<uintptr_t>(dst);
            const int32_t qbase = (int32_t)((ab & ~15ull) - ab);  // unit-relative byte of chunk 0 (-15..0)
            const int32_t isize = (int32_t)size;
            const uint32_t nch = isize > 0 ? (uint32_t)((isize - qbase + 15) >> 4) : 0u;
            const uint8_t* bmap = lds8 + rb + R_MAP;
            // Four chunks per thread at a time (this wave's next four rounds), each
            // step done for all four before the next, so that their LDS reads are
            // independent and in flight together.  A lane's record is read with the
            // next lane's, and the next lane's window is read with the lane's own
            // when the chunk runs past the lane's end, so that a chunk crossing one
            // lane boundary (the common case) takes no extra step.
            constexpr int NK = 4;
            const uint32_t c_last = nch - 1;
            const bool first_partial = qbase < 0, last_partial = nch && qbase + 16 * (int32_t)nch > isize;
            for (uint32_t cr = 64 * pw; cr < nch; cr += 64 * NPK * NK) {
                int32_t q[NK], pk[NK], qe[NK], Ln[NK];
                uint2 r0[NK], r1[NK];
                bool act[NK];
                uint4 v[NK];
#pragma unroll
                for (int k = 0; k < NK; k++) {
                    const uint32_t c = cr + 64 * NPK * k + j;
                    act[k] = c < nch;
                    q[k] = qbase + 16 * (int32_t)c;
                    pk[k] = act[k] ? max(q[k], 0) : 0;
                    qe[k] = act[k] ? min(q[k] + 16, isize) : 0;
                    Ln[k] = bmap[pk[k] >> 6];
                }
#pragma unroll
                for (int k = 0; k < NK; k++) {
                    r0[k] = lrec[Ln[k]];
                    r1[k] = lrec[min(Ln[k] + 1, 255)];
                }
                // lanes that end at or before the chunk's first byte (short lanes in the
                // chunk's 64-byte block before it)
#pragma unroll
                for (int k = 0; k < NK; k++)
                    while ((int32_t)r0[k].y <= pk[k]) {
                        Ln[k]++;
                        r0[k] = r1[k];
                        r1[k] = lrec[min(Ln[k] + 1, 255)];
                    }
                bool cross[NK];
                uint4 w[NK];
#pragma unroll
                for (int k = 0; k < NK; k++) {
                    v[k] = lds_read16(lds8, (uint32_t)((int32_t)r0[k].x + q[k]));
                    cross[k] = (int32_t)r0[k].y < qe[k] && Ln[k] < 255;
                    if (cross[k]) w[k] = lds_read16(lds8, (uint32_t)((int32_t)r1[k].x + q[k]));
                }
#pragma unroll
                for (int k = 0; k < NK; k++)
                    if (cross[k]) {
                        v[k] = merge16_from(v[k], w[k], (uint32_t)((int32_t)r0[k].y - q[k]));
                        Ln[k]++;
                    }
                // bytes past lane Ln's end (the next lane was empty or short): the
                // following non-empty lanes one by one
                for (;;) {
                    bool more = false;
#pragma unroll
                    for (int k = 0; k < NK; k++) {
                        const int32_t from = (int32_t)(cross[k] ? r1[k].y : r0[k].y);  // end of lane Ln
                        if (act[k] && from < qe[k] && Ln[k] < 255) {
                            r1[k] = lrec[++Ln[k]];
                            cross[k] = true;
                            if ((int32_t)r1[k].y > from)
                                v[k] = merge16_from(v[k], lds_read16(lds8, (uint32_t)((int32_t)r1[k].x + q[k])),
                                                    (uint32_t)(from - q[k]));
                            more = true;
                        }
                    }
                    if (__ballot(more) == 0) break;
                }
#pragma unroll
                for (int k = 0; k < NK; k++) {
                    // derived from dst (not from an integer address) so that the stores
                    // stay global: a flat store would also count against the next LDS wait
                    nchunks += act[k] ? 1u : 0u;
                    if (act[k] && q[k] >= 0 && q[k] + 16 <= isize) *reinterpret_cast<uint4*>(dst + q[k]) = v[k];
                    // the unit's first and last chunks are shared with the neighbouring
                    // units: their bytes inside this unit go out as one byte store spread
                    // over 16 lanes (lane b stores byte b), from the owner lane's registers
                    const uint32_t c0 = cr + 64 * NPK * k;
                    auto spread = [&](uint32_t owner) {
                        const int32_t qq = qbase + 16 * (int32_t)(c0 + owner);
                        const uint32_t x0 = __builtin_amdgcn_readlane(v[k].x, owner);
                        const uint32_t x1 = __builtin_amdgcn_readlane(v[k].y, owner);
                        const uint32_t x2 = __builtin_amdgcn_readlane(v[k].z, owner);
                        const uint32_t x3 = __builtin_amdgcn_readlane(v[k].w, owner);
                        const uint32_t wd = j < 4 ? x0 : (j < 8 ? x1 : (j < 12 ? x2 : x3));
                        const int32_t b = qq + (int32_t)j;
                        if (j < 16 && b >= 0 && b < isize) dst[b] = (uint8_t)(wd >> (8 * (j & 3)));
                    };
                    if (first_partial && c0 == 0) spread(0);
                    if (last_partial && c0 <= c_last && c_last < c0 + 64 && !(first_partial && c_last == 0))
                        spread(c_last - c0);
                }
            }
        }
        const uint64_t t_packed = phase ? wall_clock64() : 0;
        pbar_sync();  // every packer is done with the set
        if (pw == 0) {
            ws_signal(&pc.freed[s], 1u, j);
            if (phase && j == 0) {
                uint64_t* ph = phase + 8 * (uint64_t)u;
                ph[3] = t_seen; ph[4] = t_off; ph[5] = t_packed; ph[6] = wall_clock64(); ph[7] = nchunks;
            }
        }
    }
}


template <int SPE, bool ESC, bool SIDE, int PAIRS, int NPK, bool LIST = false>
__global__ void __launch_bounds__(64 * (2 + NPK) * PAIRS) __attribute__((amdgpu_waves_per_eu(4)))
encode_fast_kernel(const uint8_t* __restrict__ src, EncodeGeom g, const EncSym* __restrict__ d_enc,
                   const uint32_t* __restrict__ canon, FastEncParams fp, ckr_stream_header* __restrict__ hdrs,
                   uint8_t* __restrict__ sidecar, uint8_t* __restrict__ out, uint64_t* __restrict__ unit_off,
                   uint64_t* __restrict__ status, uint32_t* __restrict__ ctl, uint32_t* __restrict__ redo_list,
                   uint64_t* __restrict__ phase, const uint32_t* __restrict__ dsl) {
    encode_fast_body<SPE, ESC, SIDE, PAIRS, NPK, LIST>(src, g, d_enc, canon, fp, hdrs, sidecar, out, unit_off, status,
                                                       ctl, redo_list, phase, dsl);
}

// Several tensors' fast encodes in one launch (a shard of small tensors): the
// workgroups are shared out in proportion to the jobs' units, workgroup b
// working for the last job whose first workgroup is <= b, each job with its
// own tickets, look-back and outputs.  One launch instead of one per tensor,
// and no tensor waits for another's workgroups to leave the CUs.
template <int SPE, bool SIDE, int PAIRS, int NPK>
__global__ void __launch_bounds__(64 * (2 + NPK) * PAIRS) __attribute__((amdgpu_waves_per_eu(4)))
encode_fast_multi_kernel(FastJobs J) {
    uint32_t k = 0;
    while (k + 1 < J.n && J.j[k + 1].wg0 <= blockIdx.x) k++;
    const FastJob& b = J.j[k];
    FastEncParams fp;
    fp.sl0 = b.sl0; fp.sl1 = b.sl1; fp.cw = b.cw; fp.canon_bytes = b.canon_bytes;
    fp.stride0 = slot_stride(b.sl0); fp.stride1 = slot_stride(b.sl1);
    encode_fast_body<SPE, false, SIDE, PAIRS, NPK, false>(b.src, b.g, b.enc, b.canon, fp, b.hdrs, b.sidecar, b.out,
                                                          b.unit_off, b.status, b.ctl, b.redo, nullptr, b.dsl);
}

uint64_t encode_fast_status_words(uint64_t n_units) { return n_units + 2 * ((n_units + 63) / 64); }

// Coder pairs per workgroup that fit the LDS limit (0: none).
static uint32_t fast_enc_pairs(const FastEncParamsHost& p, uint32_t lds_limit) {
    for (uint32_t pairs = 2; pairs >= 1; pairs--)
        if (ws_lds_bytes(pairs, p.canon_bytes, slot_stride(p.sl0), slot_stride(p.sl1)) <= lds_limit) return pairs;
    return 0;
}

uint32_t encode_fast_lds_bytes(const FastEncParamsHost& p, uint32_t lds_limit) {
    const uint32_t pairs = fast_enc_pairs(p, lds_limit);
    return pairs ? ws_lds_bytes(pairs, p.canon_bytes, slot_stride(p.sl0), slot_stride(p.sl1)) : 0u;
}

hipError_t launch_encode_fast(const uint8_t* src, const EncodeGeom& g, const EncSym* d_enc, const uint32_t* canon,
                              const FastEncParamsHost& hp, uint32_t lds_limit, ckr_stream_header* hdrs,
                              uint8_t* sidecar, uint8_t* out, uint64_t* unit_off, uint64_t* status, uint32_t* ctl,
                              uint32_t* redo_list, hipStream_t s, const uint32_t* dsl) {
    uint64_t* phase = prof_phase_buffer(g.n_units * 8, s);
    FastEncParams fp;
    fp.sl0 = hp.sl0; fp.sl1 = hp.sl1; fp.cw = hp.cw; fp.canon_bytes = hp.canon_bytes;
    fp.stride0 = slot_stride(hp.sl0); fp.stride1 = slot_stride(hp.sl1);
    const uint32_t pairs = fast_enc_pairs(hp, lds_limit);
    if (!pairs) return hipErrorInvalidValue;
    const uint32_t lb = ws_lds_bytes(pairs, fp.canon_bytes, fp.stride0, fp.stride1);
    const uint64_t n = g.n_units;
    hipError_t e = hipSuccess;
    // persistent grid: as many workgroups as fit on the device at once (more
    // would only find the tickets gone), never more than the units need
    int dev = 0, ncu = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    auto run = [&](auto kern, uint32_t nthreads) -> hipError_t {
        const void* kf = reinterpret_cast<const void*>(kern);
        hipError_t r = hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lb);
        if (r != hipSuccess) return r;
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, nthreads, lb) != hipSuccess || per_cu < 1)
            per_cu = 1;
        const uint64_t need = (n + pairs - 1) / pairs;
        const uint32_t grid = (uint32_t)std::min<uint64_t>(need, (uint64_t)per_cu * (uint64_t)std::max(ncu, 1));
        CKR_LAUNCH("encode_fast_kernel", s,
                   kern<<<grid, nthreads, lb, s>>>(src, g, d_enc, canon, fp, hdrs, sidecar, out, unit_off, status,
                                                   ctl, redo_list, phase, dsl));
        return hipGetLastError();
    };
#define CKR_FAST_ENC_P(SPE_, ESC_, SIDE_, NPK_)                                                                  \
    (pairs == 2 ? run(encode_fast_kernel<SPE_, ESC_, SIDE_, 2, NPK_>, 128u * (2 + NPK_))                           \
                : run(encode_fast_kernel<SPE_, ESC_, SIDE_, 1, NPK_>, 64u * (2 + NPK_)))
#define CKR_FAST_ENC(SPE_, ESC_, SIDE_) CKR_FAST_ENC_P(SPE_, ESC_, SIDE_, ENC_NPK)
    const bool side = sidecar != nullptr;
    if (g.spe == 2) {
        if (hp.escapes) e = side ? CKR_FAST_ENC(2, true, true) : CKR_FAST_ENC(2, true, false);
        else e = side ? CKR_FAST_ENC(2, false, true) : CKR_FAST_ENC(2, false, false);
    } else {
        if (hp.escapes) e = side ? CKR_FAST_ENC(1, true, true) : CKR_FAST_ENC(1, true, false);
        else e = side ? CKR_FAST_ENC(1, false, true) : CKR_FAST_ENC(1, false, false);
    }
#undef CKR_FAST_ENC
#undef CKR_FAST_ENC_P
    return e;
}

hipError_t launch_encode_fast_multi(const FastJob* jobs, uint32_t n, uint32_t lds_limit, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (n > kMaxFastJobs) return hipErrorInvalidValue;
    const int spe = jobs[0].g.spe;
    const bool side = jobs[0].sidecar != nullptr;
    uint32_t pairs = 2, lb = 0;
    uint64_t units = 0;
    for (uint32_t i = 0; i < n; i++) {
        if (jobs[i].g.spe != spe || (jobs[i].sidecar != nullptr) != side || (spe != 1 && spe != 2))
            return hipErrorInvalidValue;
        const FastEncParamsHost hp{jobs[i].sl0, jobs[i].sl1, jobs[i].cw, jobs[i].canon_bytes, false};
        const uint32_t pj = fast_enc_pairs(hp, lds_limit);
        if (!pj) return hipErrorInvalidValue;
        pairs = std::min(pairs, pj);
        units += jobs[i].g.n_units;
    }
    for (uint32_t i = 0; i < n; i++)
        lb = std::max(lb, ws_lds_bytes(pairs, jobs[i].canon_bytes, slot_stride(jobs[i].sl0), slot_stride(jobs[i].sl1)));
    int dev = 0, ncu = 0;
    hipError_t e;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    auto run = [&](auto kern, uint32_t nthreads) -> hipError_t {
        hipError_t r = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lb);
        if (r != hipSuccess) return r;
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, nthreads, lb) != hipSuccess || per_cu < 1)
            per_cu = 1;
        // workgroups in proportion to the jobs' units (rounded up, so that a small
        // job is not left behind), never more than a job's units need
        const uint64_t slots = (uint64_t)per_cu * (uint64_t)std::max(ncu, 1);
        FastJobs J{};
        J.n = n;
        uint32_t wg = 0;
        for (uint32_t i = 0; i < n; i++) {
            J.j[i] = jobs[i];
            const uint64_t need = (jobs[i].g.n_units + pairs - 1) / pairs;
            const uint64_t share = units ? (slots * jobs[i].g.n_units + units - 1) / units : 1;
            J.j[i].wg0 = wg;
            wg += (uint32_t)std::max<uint64_t>(1, std::min(need, share));
        }
        CKR_LAUNCH("encode_fast_kernel", s, kern<<<wg, nthreads, lb, s>>>(J));
        return hipGetLastError();
    };
    if (spe == 2)
        return pairs == 2 ? (side ? run(encode_fast_multi_kernel<2, true, 2, ENC_NPK>, 128u * (2 + ENC_NPK))
                                  : run(encode_fast_multi_kernel<2, false, 2, ENC_NPK>, 128u * (2 + ENC_NPK)))
                          : (side ? run(encode_fast_multi_kernel<2, true, 1, ENC_NPK>, 64u * (2 + ENC_NPK))
                                  : run(encode_fast_multi_kernel<2, false, 1, ENC_NPK>, 64u * (2 + ENC_NPK)));
    return pairs == 2 ? (side ? run(encode_fast_multi_kernel<1, true, 2, ENC_NPK>, 128u * (2 + ENC_NPK))
                              : run(encode_fast_multi_kernel<1, false, 2, ENC_NPK>, 128u * (2 + ENC_NPK)))
                      : (side ? run(encode_fast_multi_kernel<1, true, 1, ENC_NPK>, 64u * (2 + ENC_NPK))
                              : run(encode_fast_multi_kernel<1, false, 1, ENC_NPK>, 64u * (2 + ENC_NPK)));
}

// The redo list of a launch_encode_fast launch (ctl[1] units, queued once the
// host has seen that there are some): one coder pair per workgroup with slots
// of 2 bytes per row (any lane fits), one workgroup per CU.
static uint32_t encode_fast_list_slot(const EncodeGeom& g) {
    return (uint32_t)(2 * ((g.unit + 255) / 256) + 8 + 3) & ~3u;
}

bool encode_fast_list_fits(const FastEncParamsHost& hp, const EncodeGeom& g, uint32_t lds_limit) {
    const uint32_t st = slot_stride(encode_fast_list_slot(g));
    return ws_lds_bytes(1, hp.canon_bytes, st, st) <= lds_limit;
}

hipError_t launch_encode_fast_list(const uint8_t* src, const EncodeGeom& g, const EncSym* d_enc, const uint32_t* canon,
                                   const FastEncParamsHost& hp, uint32_t lds_limit, ckr_stream_header* hdrs,
                                   uint8_t* out, uint64_t* unit_off, uint64_t* status, uint32_t* ctl,
                                   uint32_t* redo_list, hipStream_t s) {
    if (!encode_fast_list_fits(hp, g, lds_limit)) return hipErrorInvalidValue;
    FastEncParams fp;
    fp.sl0 = fp.sl1 = encode_fast_list_slot(g);
    fp.cw = hp.cw; fp.canon_bytes = hp.canon_bytes;
    fp.stride0 = slot_stride(fp.sl0); fp.stride1 = slot_stride(fp.sl1);
    const uint32_t lb = ws_lds_bytes(1, fp.canon_bytes, fp.stride0, fp.stride1);
    int dev = 0, ncu = 0;
    hipError_t e;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    auto run = [&](auto kern) -> hipError_t {
        const uint32_t nthreads = 64u * (2 + ENC_NPK);
        hipError_t r = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lb);
        if (r != hipSuccess) return r;
        const uint32_t grid = (uint32_t)std::min<uint64_t>(g.n_units, (uint64_t)std::max(ncu, 1));
        CKR_LAUNCH("encode_fast_redo_kernel", s,
                   kern<<<grid, nthreads, lb, s>>>(src, g, d_enc, canon, fp, hdrs, nullptr, out, unit_off, status, ctl,
                                                   redo_list, nullptr, nullptr));
        return hipGetLastError();
    };
    if (g.spe == 2) return hp.escapes ? run(encode_fast_kernel<2, true, false, 1, ENC_NPK, true>)
                                      : run(encode_fast_kernel<2, false, false, 1, ENC_NPK, true>);
    return hp.escapes ? run(encode_fast_kernel<1, true, false, 1, ENC_NPK, true>)
                      : run(encode_fast_kernel<1, false, false, 1, ENC_NPK, true>);
}

// ------------------------------------------------------------------ large units: two passes
// Units of more than 256 rows (above 64 KiB) of masked dtypes.  A lane's
// stream is one serial state chain over every row of its unit, but running the
// chain needs none of its output.  Pass 1 (seg_size_kernel, one wave per unit)
// runs it for both live lanes of every column, counting renorm bytes, and
// records each lane's state and byte count at the entry of every SEG_ROWS-row
// segment; at the end it knows every lane's size, so it writes the headers
// (lane offsets, passthrough decision) and the unit size.  After the scan of
// unit sizes, pass 2 (seg_code_kernel, one wave per segment) codes every
// segment from its recorded state straight into its place: within a lane's
// stream, segment s's bytes are [total - E(s-1), total - E(s)) from its start,
// E(s) being the bytes the rows above segment s emit, E(-1) = total.  No lane
// scratch, and units x segments independent work items.
static constexpr uint32_t SEG_ROWS = 256;

__host__ __device__ constexpr uint32_t seg_count(uint64_t unit) {
    return (uint32_t)((unit + 256ull * SEG_ROWS - 1) / (256ull * SEG_ROWS));
}

// enc_step's state update without the bytes: returns how many it emits.
template <bool ESC>
__device__ __forceinline__ uint32_t seg_size_step(uint32_t& x, uint4 t) {
    const uint32_t f8 = t.w;
    uint32_t n = ((x >> 24) >= f8) ? 2u : (((x >> 16) >= f8) ? 1u : 0u);
    const uint32_t xr = x >> (8u * n);
    const uint32_t q = __umulhi(xr, t.x) >> (t.y >> 24);
    const uint32_t xn = xr + t.z + __umul24(q, t.y);
    if (ESC) {
        const bool esc = f8 == 0u;
        n = esc ? 1u : n;
        x = esc ? x : xn;
    } else {
        x = xn;
    }
    return n;
}

__device__ __forceinline__ void seg_load_table(uint4* tab, const EncSym* d_enc) {
    const uint4 tv = reinterpret_cast<const uint4*>(d_enc)[threadIdx.x];
    const EncSym e = {tv.x, tv.y, tv.z, tv.w};
    tab[threadIdx.x] = enc_quad(e);
}

// Index (0..2) of the canonical entry for K symbols (see canon_entry).
__device__ __forceinline__ uint32_t canon_index(const uint32_t* canon, uint32_t cw, uint32_t K) {
    return canon[0] == K ? 0u : (canon[4 + cw] == K ? 1u : 2u);
}

// Checkpoint records: rec[((u * S + s) * 2 + p) * 64 + j] = {state, bytes
// emitted so far} of live lane p (0: byte FL, 1: byte 3) of column j at the
// entry of segment s (before its top row is coded).
template <int SPE, bool ESC>
__global__ void __launch_bounds__(256) seg_size_kernel(const uint8_t* __restrict__ src, EncodeGeom g,
                                                       const EncSym* __restrict__ d_enc,
                                                       const uint32_t* __restrict__ canon, uint32_t cw, uint32_t S,
                                                       uint2* __restrict__ rec, ckr_stream_header* __restrict__ hdrs,
                                                       uint32_t* __restrict__ unit_size, uint32_t* __restrict__ err) {
    __shared__ uint4 tab[256];
    seg_load_table(tab, d_enc);
    if (blockIdx.x == 0 && threadIdx.x == 0) *err = 0;  // pass 2 runs after this grid
    __syncthreads();
    constexpr int FL = SPE == 2 ? 2 : 1;
    constexpr uint32_t SH0 = 8u * FL;
    const uint32_t j = threadIdx.x & 63;
    const uint64_t u = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (u >= g.n_units) return;
    const uint64_t ubase = u * g.unit;
    const uint32_t len = (uint32_t)((g.n_bytes - ubase < g.unit) ? (g.n_bytes - ubase) : g.unit);
    const uint32_t kf = len >> 8, r = len & 255u, K = kf + (r ? 1u : 0u);
    uint32_t x0 = L, x1 = L, e0 = 0, e1 = 0;
    uint2* ur = rec + u * S * 128 + j;
    auto record = [&](uint32_t s) {
        ur[s * 128] = make_uint2(x0, e0);
        ur[s * 128 + 64] = make_uint2(x1, e1);
    };
    record((K - 1) / SEG_ROWS);
    if (r) {  // the tensor's partial top row: lane 4j + b holds a byte when 4j + b < r
        const uint8_t* p = src + ubase + 256ull * kf + 4 * j;
        if (4 * j + FL < r) e0 += seg_size_step<ESC>(x0, tab[p[FL]]);
        if (4 * j + 3 < r) e1 += seg_size_step<ESC>(x1, tab[p[3]]);
        if (kf && kf % SEG_ROWS == 0) record(kf / SEG_ROWS - 1);
    }
    const uint32_t* in32 = reinterpret_cast<const uint32_t*>(src + ubase) + j;  // row k at in32[64 k]
    const uint32_t ng = kf >> 5;
    for (int32_t k = (int32_t)kf - 1; k >= (int32_t)(32 * ng); k--) {
        const uint32_t wd = in32[64 * k];
        const uint4 t0 = tab[(wd >> SH0) & 255u], t1 = tab[wd >> 24];
        e0 += seg_size_step<ESC>(x0, t0);
        e1 += seg_size_step<ESC>(x1, t1);
        if (k && k % SEG_ROWS == 0) record(k / SEG_ROWS - 1);
    }
    if (ng) {
        // groups of 32 rows from the top down, the next group's loads in flight
        // while the current one is coded; table entries read 4 rows ahead
        auto load = [&](uint32_t (&rr)[32], uint32_t gi) {
            const uint32_t* p = in32 + 64 * (32 * gi + 31);
#pragma unroll
            for (int i = 0; i < 32; i++) rr[i] = p[-64 * i];
        };
        auto code = [&](const uint32_t (&rr)[32], uint32_t gi) {
            uint4 ta[2][4], tb[2][4];
            auto fetch = [&](int buf, int i0) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    ta[buf][i] = tab[(rr[i0 + i] >> SH0) & 255u];
                    tb[buf][i] = tab[rr[i0 + i] >> 24];
                }
            };
            fetch(0, 0);
#pragma unroll
            for (int bt = 0; bt < 8; bt++) {
                if (bt < 7) fetch((bt + 1) & 1, 4 * (bt + 1));
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    e0 += seg_size_step<ESC>(x0, ta[bt & 1][i]);
                    e1 += seg_size_step<ESC>(x1, tb[bt & 1][i]);
                }
            }
            const uint32_t k = 32 * gi;  // the row just coded
            if (k && k % SEG_ROWS == 0) record(k / SEG_ROWS - 1);
        };
        uint32_t ra[32], rb[32];
        uint32_t gi = ng - 1;
        load(ra, gi);
        for (;;) {
            if (gi == 0) { code(ra, 0); break; }
            load(rb, gi - 1);
            code(ra, gi);
            gi--;
            if (gi == 0) { code(rb, 0); break; }
            load(ra, gi - 1);
            code(rb, gi);
            gi--;
        }
    }
    // headers: the live lanes' sizes and final states, the zero-plane lanes'
    // canonical ones; lane offsets by a wave scan; passthrough when the packed
    // unit would not be smaller (ANSCompressor.cpp:694-713)
    uint32_t c[4], fs[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
        if (b == FL) { c[b] = e0; fs[b] = x0; }
        else if (b == 3) { c[b] = e1; fs[b] = x1; }
        else {
            const uint32_t Kb = kf + ((4 * j + b < r) ? 1u : 0u);
            const uint32_t* ce = canon_entry(canon, cw, Kb);
            fs[b] = ce[1];
            c[b] = ce[2];
        }
    }
    const uint32_t tsum = c[0] + c[1] + c[2] + c[3];
    uint32_t incl = tsum;
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
        const uint32_t v = __shfl_up(incl, d, 64);
        if (j >= d) incl += v;
    }
    const uint32_t total = __shfl(incl, 63, 64);
    const bool raw = total >= len;
    uint32_t off = incl - tsum;
    ckr_stream_header* uh = hdrs + u * 256 + 4 * j;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        ckr_stream_header h;
        h.final_state = raw ? 0u : fs[b];
        h.byte_count = raw ? ((j == 0 && b == 0) ? len : 0u) : c[b];
        h.buf_offset = raw ? 0u : off;
        h.pad = 0;
        uh[b] = h;
        off += c[b];
    }
    if (j == 0) unit_size[u] = raw ? len : total;
}

// A live lane of pass 2: the coder window of EncLane, whose dwords go into an
// LDS line buffer of SEG_LINE bytes indexed by their address in memory (ud +
// offset) mod SEG_LINE; a run's bytes are written to memory a whole line at a
// time (measured: dword stores straight to memory, each lane filling its line
// over ~100 rows, wrote 4.4x the bytes out of L2).  The run's end e
// may be unaligned: a = -e mod 4 (in memory) phantom bytes prime the window, so
// every flush is an aligned dword.  A store that is not a flush (fewer than 4
// bytes pending) lands in the buffer at the next dword, which a later flush
// overwrites (or which the final copy does not read).
static constexpr uint32_t SEG_LINE = 64;  // bytes a line buffer holds (a multiple of 16)

struct SegLane {
    EncLane c;
    int32_t go;    // next dword to flush (offset from the unit's output base, aligned in memory)
    int32_t rs;    // the run's first byte
    int32_t e;     // one past its last byte
    int32_t lc;    // start of the lowest line written out (e until one is)
    uint32_t lb;   // LDS byte address of the line buffer
};

__device__ __forceinline__ void seg_lane_init(SegLane& l, uint32_t x, int32_t rs, int32_t e, uint32_t ua, uint32_t lb) {
    const uint32_t a = (0u - (ua + (uint32_t)e)) & 3u;
    l.c.x = x;
    l.c.hi = 0;
    l.c.lo = 0;
    l.c.sel = 0x08090A0Bu - a * 0x01010101u;
    l.c.ptr = 0;
    l.go = e + (int32_t)a - 4;
    l.rs = rs;
    l.e = e;
    l.lc = e;
    l.lb = lb;
}

// Bytes [lo, hi) of one line (offsets from ud) from the lane's line buffer to
// memory: dword stores where a whole aligned dword is inside, byte stores else.
__device__ __attribute__((noinline)) void seg_line_bytes(const uint8_t* lds8, uint32_t lb, uint32_t ua, uint8_t* ud,
                                                         int32_t lo, int32_t hi) {
    for (int32_t d = lo - (int32_t)((ua + (uint32_t)lo) & 3u); d < hi; d += 4) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(lds8 + lb + ((ua + (uint32_t)d) & (SEG_LINE - 1)));
        if (d >= lo && d + 4 <= hi) *reinterpret_cast<uint32_t*>(ud + d) = v;
        else
            for (int32_t b = 0; b < 4; b++)
                if (d + b >= lo && d + b < hi) ud[d + b] = (uint8_t)(v >> (8 * b));
    }
}

// One flush.  Returns the line start (offset) when this flush completed a
// line (wrote its first dword), else INT32_MIN.
__device__ __forceinline__ int32_t seg_flush(SegLane& l, uint8_t* lds8, uint32_t ua) {
    const uint32_t v = __builtin_amdgcn_perm(l.c.hi, l.c.lo, l.c.sel);
    const bool fl = (l.c.sel & 8u) == 0u;
    const uint32_t o = (ua + (uint32_t)l.go) & (SEG_LINE - 1);
    *reinterpret_cast<uint32_t*>(lds8 + l.lb + o) = v;
    const int32_t done = (fl && o == 0u) ? l.go : INT32_MIN;
    l.go -= fl ? 4 : 0;
    l.c.sel += fl ? 0x04040404u : 0u;
    return done;
}

// After the flushes of a step: lines completed by them go out.  A line wholly
// inside its run goes out as 16-byte stores, the wave copying 64 / (SEG_LINE /
// 16) such lines per round; the run's top line, which shares bytes with the
// next run, goes out byte-exact by its own thread.
struct SegCopyEnt { uint32_t lb; int32_t g; };
__device__ __forceinline__ void seg_lines_out(SegLane& l0, SegLane& l1, int32_t d0, int32_t d1, uint8_t* lds8,
                                              SegCopyEnt* tbl, uint32_t ua, uint8_t* ud, uint32_t j) {
    const bool f0 = d0 != INT32_MIN && d0 + (int32_t)SEG_LINE <= l0.e;
    const bool f1 = d1 != INT32_MIN && d1 + (int32_t)SEG_LINE <= l1.e;
    if (d0 != INT32_MIN) { if (!f0) seg_line_bytes(lds8, l0.lb, ua, ud, d0, l0.e); l0.lc = d0; }
    if (d1 != INT32_MIN) { if (!f1) seg_line_bytes(lds8, l1.lb, ua, ud, d1, l1.e); l1.lc = d1; }
    const uint64_t m0 = __ballot(f0), m1 = __ballot(f1);
    if ((m0 | m1) == 0) return;
    const uint32_t n0 = (uint32_t)__popcll(m0), n = n0 + (uint32_t)__popcll(m1);
    const uint64_t below = (1ull << j) - 1ull;
    if (f0) tbl[__popcll(m0 & below)] = SegCopyEnt{l0.lb, d0};
    if (f1) tbl[n0 + __popcll(m1 & below)] = SegCopyEnt{l1.lb, d1};
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    constexpr uint32_t TPL = SEG_LINE / 16;  // threads per line
    for (uint32_t k0 = 0; k0 < n; k0 += 64 / TPL) {
        const uint32_t k = k0 + j / TPL, c = j % TPL;
        if (k < n) {
            const SegCopyEnt t = tbl[k];
            const uint4 v = *reinterpret_cast<const uint4*>(lds8 + t.lb + 16 * c);
            *reinterpret_cast<uint4*>(ud + t.g + 16 * c) = v;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// End of the item: the last flush, the pending bytes (the run's first ones)
// into the buffer, and the bytes below the lowest line written out.  True when
// they end exactly at the run start.
__device__ __forceinline__ bool seg_finish_lane(SegLane& l, uint8_t* lds8, uint32_t ua, uint8_t* ud) {
    const uint32_t P = 0x0Bu - (l.c.sel & 0xFFu);  // < 4 after the last flush
    const uint32_t v = __builtin_amdgcn_perm(l.c.hi, l.c.lo, l.c.sel);  // its top P bytes
    *reinterpret_cast<uint32_t*>(lds8 + l.lb + ((ua + (uint32_t)l.go) & (SEG_LINE - 1))) = v;
    const bool ok = l.go + 4 - (int32_t)P == l.rs && l.lc - l.rs <= (int32_t)SEG_LINE;
    if (ok && l.rs < l.lc) seg_line_bytes(lds8, l.lb, ua, ud, l.rs, l.lc);
    return ok;
}

// n bytes of a dword-aligned byte stream (readable for one dword past its end)
// to dst by one thread: aligned dword stores, byte stores at the two ends.
__device__ __forceinline__ void seg_copy_thread(uint8_t* dst, const uint32_t* src32, uint32_t n) {
    if (n == 0) return;
    const uint32_t lead = (uint32_t)(reinterpret_cast<uintptr_t>(dst) & 3u);
    uint8_t* d0 = dst - lead;
    const uint32_t nd = (lead + n + 3) >> 2;  // src32[0 .. nd) are read: nd - 1 <= (n + 2) / 4
    // dword i of dst's aligned span holds stream bytes 4i - lead .. 4i - lead + 3
    uint32_t prev = 0;
    for (uint32_t i0 = 0; i0 < nd; i0 += 8) {
        uint32_t w[8];
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) w[k] = i0 + k < nd ? src32[i0 + k] : 0u;
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) {
            const uint32_t i = i0 + k;
            if (i >= nd) break;
            const uint32_t v = lead ? __builtin_amdgcn_alignbyte(w[k], prev, 4u - lead) : w[k];
            const uint32_t b1 = 4 * i + 4 <= lead + n ? 4u : lead + n - 4 * i;
            if ((i > 0 || lead == 0) && b1 == 4) *reinterpret_cast<uint32_t*>(d0 + 4 * i) = v;
            else
                for (uint32_t b = (i == 0 ? lead : 0u); b < b1; b++) d0[4 * i + b] = (uint8_t)(v >> (8 * b));
            prev = w[k];
        }
    }
}

// An item of pass 2 by list: unit u, segments [sg & 0xFFFF, + sg >> 16).
struct SegItem {
    uint32_t u, sg;
};

// LDS of seg_code_kernel: table | per wave: 128 line buffers of SEG_LINE bytes, then
// 128 copy-table entries.
static constexpr uint32_t SEG_WAVE_LDS = 128 * SEG_LINE + 128 * 8;
static constexpr uint32_t SEG_LDS = 4096 + 4 * SEG_WAVE_LDS;

// Pass 2 for one item, G consecutive segments [s0, s0 + G) of unit u, coded by
// one wave from the top of segment s0 + G - 1 down (wv: the wave's index in
// its workgroup, which selects its LDS buffers).
template <int SPE, bool ESC>
__device__ void seg_code_item(const uint8_t* __restrict__ src, const EncodeGeom& g,
                              const uint32_t* __restrict__ canon, uint32_t cw, uint32_t S, uint32_t G,
                              const uint2* __restrict__ rec, const ckr_stream_header* __restrict__ hdrs,
                              const uint32_t* __restrict__ unit_size, const uint64_t* __restrict__ unit_off,
                              uint8_t* __restrict__ sidecar, uint8_t* __restrict__ out, uint32_t* __restrict__ aux,
                              uint64_t u, uint32_t s0, uint32_t wv, const uint4* tab, uint8_t* lds8) {
    constexpr int FL = SPE == 2 ? 2 : 1;
    constexpr uint32_t SH0 = 8u * FL;
    const uint32_t j = threadIdx.x & 63;
    if (u >= g.n_units) return;
    const uint64_t ubase = u * g.unit;
    const uint32_t len = (uint32_t)((g.n_bytes - ubase < g.unit) ? (g.n_bytes - ubase) : g.unit);
    const uint32_t kf = len >> 8, r = len & 255u, K = kf + (r ? 1u : 0u);
    const uint32_t Su = (K + SEG_ROWS - 1) / SEG_ROWS;
    if (s0 >= Su) return;
    const uint32_t s1 = min(s0 + G, Su) - 1;  // top segment of the item
    const uint32_t lo = s0 * SEG_ROWS, hi = min((s1 + 1) * SEG_ROWS, K), fhi = min(hi, kf);
    const bool ptop = r && hi == K;  // the partial row kf is the item's top row
    uint8_t* ud = out + unit_off[u];
    const uint32_t ua = (uint32_t)reinterpret_cast<uintptr_t>(ud);
    const ckr_stream_header* uh = hdrs + u * 256;
    const bool raw = unit_size[u] >= len;
    const uint32_t* in32 = reinterpret_cast<const uint32_t*>(src + ubase) + j;  // row k at in32[64 k]
    uint16_t* sc16 = reinterpret_cast<uint16_t*>(sidecar + (ubase >> 1) + 2 * j);  // row k at sc16[64 k]
    auto side = [&](uint32_t k, uint32_t wd) {
        sc16[64 * k] = (uint16_t)(SPE == 2 ? (wd & 0xFFFFu) : ((wd & 0xFFu) | ((wd >> 8) & 0xFF00u)));
    };
    const uint32_t lm = live_mask32<SPE>();
    if (raw) {  // passthrough: the masked bytes, and the sidecar
        const bool al = (ua & 3u) == 0;
        for (uint32_t k = lo; k < fhi; k++) {
            const uint32_t wd = in32[64 * k];
            side(k, wd);
            uint8_t* d = ud + 256 * k + 4 * j;
            if (al) *reinterpret_cast<uint32_t*>(d) = wd & lm;
            else
                for (int b = 0; b < 4; b++) d[b] = (uint8_t)((wd & lm) >> (8 * b));
        }
        if (ptop && 4 * j < r) {
            const uint8_t* p = src + ubase + 256ull * kf + 4 * j;
            const uint32_t nv = min(r - 4 * j, 4u);
            uint32_t wd = 0;
            for (uint32_t b = 0; b < nv; b++) wd |= (uint32_t)p[b] << (8 * b);
            write_sidecar_row<SPE>(sidecar, ubase + 256ull * kf + 4 * j, wd, nv);
            for (uint32_t b = 0; b < nv; b++) ud[256 * kf + 4 * j + b] = (uint8_t)((wd & lm) >> (8 * b));
        }
        return;
    }
    const uint32_t wbase = 4096 + wv * SEG_WAVE_LDS;
    SegCopyEnt* tbl = reinterpret_cast<SegCopyEnt*>(lds8 + wbase + 128 * SEG_LINE);
    {
        const ckr_stream_header h0 = uh[4 * j + FL], h1 = uh[4 * j + 3];
        const uint2* rp = rec + (u * S + s1) * 128 + j;  // entry of the top segment
        const uint2 c0 = rp[0], c1 = rp[64];
        uint2 n0, n1;  // state and bytes after the item
        if (s0) {
            const uint2* rq = rec + (u * S + s0 - 1) * 128 + j;
            n0 = rq[0];
            n1 = rq[64];
        } else {
            n0 = make_uint2(h0.final_state, h0.byte_count);
            n1 = make_uint2(h1.final_state, h1.byte_count);
        }
        SegLane l0, l1;
        seg_lane_init(l0, c0.x, (int32_t)(h0.buf_offset + h0.byte_count - n0.y),
                      (int32_t)(h0.buf_offset + h0.byte_count - c0.y), ua, wbase + SEG_LINE * j);
        seg_lane_init(l1, c1.x, (int32_t)(h1.buf_offset + h1.byte_count - n1.y),
                      (int32_t)(h1.buf_offset + h1.byte_count - c1.y), ua, wbase + SEG_LINE * (64 + j));
        auto flush2 = [&]() {
            const int32_t d0 = seg_flush(l0, lds8, ua);
            const int32_t d1 = seg_flush(l1, lds8, ua);
            seg_lines_out(l0, l1, d0, d1, lds8, tbl, ua, ud, j);
        };
        if (ptop) {
            const uint8_t* p = src + ubase + 256ull * kf + 4 * j;
            if (4 * j < r) {
                const uint32_t nv = min(r - 4 * j, 4u);
                uint32_t wd = 0;
                for (uint32_t b = 0; b < nv; b++) wd |= (uint32_t)p[b] << (8 * b);
                write_sidecar_row<SPE>(sidecar, ubase + 256ull * kf + 4 * j, wd, nv);
            }
            if (4 * j + FL < r) { const uint32_t sy = p[FL]; enc_step<ESC>(l0.c, sy, tab[sy]); }
            if (4 * j + 3 < r) { const uint32_t sy = p[3]; enc_step<ESC>(l1.c, sy, tab[sy]); }
            flush2();
        }
        auto row = [&](uint32_t k, uint32_t wd, uint4 t0, uint4 t1) {
            side(k, wd);
            enc_step<ESC>(l0.c, (wd >> SH0) & 255u, t0);
            enc_step<ESC>(l1.c, wd >> 24, t1);
        };
        const uint32_t nf = fhi - lo, ng = nf >> 4;
        for (int32_t k = (int32_t)fhi - 1; k >= (int32_t)(lo + 16 * ng); k--) {
            const uint32_t wd = in32[64 * k];
            row((uint32_t)k, wd, tab[(wd >> SH0) & 255u], tab[wd >> 24]);
            flush2();
        }
        if (ng) {
            // groups of 16 rows from the top down, the next group's loads in
            // flight while the current one is coded; table entries 2 rows ahead
            auto load = [&](uint32_t (&rr)[16], uint32_t gi) {
                const uint32_t* p = in32 + 64 * (lo + 16 * gi + 15);
#pragma unroll
                for (int i = 0; i < 16; i++) rr[i] = p[-64 * i];
            };
            auto code = [&](const uint32_t (&rr)[16], uint32_t gi) {
                const uint32_t ktop = lo + 16 * gi + 15;
                uint4 ta[2][2], tb[2][2];
                auto fetch = [&](int buf, int i0) {
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        ta[buf][i] = tab[(rr[i0 + i] >> SH0) & 255u];
                        tb[buf][i] = tab[rr[i0 + i] >> 24];
                    }
                };
                fetch(0, 0);
#pragma unroll
                for (int bt = 0; bt < 8; bt++) {
                    if (bt < 7) fetch((bt + 1) & 1, 2 * (bt + 1));
                    row(ktop - 2 * bt, rr[2 * bt], ta[bt & 1][0], tb[bt & 1][0]);
                    row(ktop - 2 * bt - 1, rr[2 * bt + 1], ta[bt & 1][1], tb[bt & 1][1]);
                    flush2();
                }
            };
            uint32_t ra[16], rb[16];
            uint32_t gi = ng - 1;
            load(ra, gi);
            for (;;) {
                if (gi == 0) { code(ra, 0); break; }
                load(rb, gi - 1);
                code(ra, gi);
                gi--;
                if (gi == 0) { code(rb, 0); break; }
                load(ra, gi - 1);
                code(rb, gi);
                gi--;
            }
        }
        flush2();
        const bool ok0 = seg_finish_lane(l0, lds8, ua, ud) && l0.c.x == n0.x;
        const bool ok1 = seg_finish_lane(l1, lds8, ua, ud) && l1.c.x == n1.x;
        if (!(ok0 && ok1)) atomicOr(aux, 1u);
    }
    // the zero-plane lanes copy their canonical stream: thread j those of
    // column j, in the unit's item j mod (items of the unit)
    const uint32_t iu = (Su + G - 1) / G;
    if (j % iu == s0 / G) {
        const uint32_t* cbytes = canon + 3 * (4 + cw);
        constexpr uint32_t ZB1 = SPE == 2 ? 1u : 2u;  // zero bytes of a column: 0 and ZB1
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t lane = 4 * j + (h ? ZB1 : 0u);
            const ckr_stream_header hz = uh[lane];
            const uint32_t Kb = kf + ((lane < r) ? 1u : 0u);
            seg_copy_thread(ud + hz.buf_offset, cbytes + canon_index(canon, cw, Kb) * cw, hz.byte_count);
        }
    }
}

// One wave per item.  Grid mode (LIST false): items of G consecutive segments
// in unit order, G segments per item.  List mode: the items in list[0,
// *list_count), each wave taking every n-th one (n: the grid's waves).
template <int SPE, bool ESC, bool LIST>
__global__ void __launch_bounds__(256) seg_code_kernel(const uint8_t* __restrict__ src, EncodeGeom g,
                                                       const EncSym* __restrict__ d_enc,
                                                       const uint32_t* __restrict__ canon, uint32_t cw, uint32_t S,
                                                       uint32_t G, const uint2* __restrict__ rec,
                                                       const ckr_stream_header* __restrict__ hdrs,
                                                       const uint32_t* __restrict__ unit_size,
                                                       const uint64_t* __restrict__ unit_off,
                                                       uint8_t* __restrict__ sidecar, uint8_t* __restrict__ out,
                                                       uint32_t* __restrict__ aux, const SegItem* __restrict__ list,
                                                       const uint32_t* __restrict__ list_count) {
    extern __shared__ uint4 seg_lds[];
    uint4* tab = seg_lds;
    uint8_t* lds8 = reinterpret_cast<uint8_t*>(seg_lds);
    seg_load_table(tab, d_enc);
    __syncthreads();
    const uint32_t wv = threadIdx.x >> 6;
    // workgroups go round-robin over the 8 XCDs: those of one XCD take
    // consecutive items, so the neighbouring runs of a lane share its L2
    const uint32_t nb = gridDim.x, q8 = nb >> 3, r8 = nb & 7u, xcd = blockIdx.x & 7u;
    const uint32_t lbk = xcd * q8 + min(xcd, r8) + (blockIdx.x >> 3);
    const uint32_t ipu = (S + G - 1) / G;  // items per unit
    const uint32_t n = LIST ? *list_count : 1u;
    const uint32_t k0 = LIST ? blockIdx.x * 4 + wv : 0u, step = LIST ? gridDim.x * 4 : 1u;
    for (uint32_t k = k0; k < n; k += step) {
        uint64_t u;
        uint32_t s0, gk;
        if constexpr (LIST) {
            const SegItem it = list[k];
            u = it.u;
            s0 = it.sg & 0xFFFFu;
            gk = it.sg >> 16;
        } else {
            const uint64_t item = (uint64_t)lbk * 4 + wv;
            u = item / ipu;
            s0 = (uint32_t)(item % ipu) * G;
            gk = G;
        }
        seg_code_item<SPE, ESC>(src, g, canon, cw, S, gk, rec, hdrs, unit_size, unit_off, sidecar, out, aux, u, s0,
                                wv, tab, lds8);
    }
}

// Pass 2 of a two-pass encode on encode_fast_kernel's coder and packer waves.
// seg_size_kernel has written every lane's {state, bytes so far} at the entry
// of each 256-row segment, the headers and the unit sizes; unit_scan_kernel
// the unit offsets.  An item is one 256-row segment (64 KiB of input; the top
// segment of a partial last unit may be shorter), taken in address order from
// a ticket counter.
// What lane l emits in segment s has a known place: with o and c its header's
// buf_offset and byte_count, B its bytes so far at the entry of s and B' the
// same at the entry of s - 1 (c for s = 0), the piece is [o + c - B', o + c -
// B) of the unit's output, B' - B bytes.  The two coder waves of a pair code
// the segment from the recorded entry states into the pair's LDS slots (sized
// for 256 rows, as for 64 KiB units) and check that every lane ends in the
// state and at the byte count the next record gives (a mismatch sets *err).
// The packer waves copy each piece to its place, 16-byte stores aligned in
// memory and byte stores at its two ends (the lines there are shared with the
// neighbouring segments' pieces, not their bytes), and copy the canonical
// streams of the unit's zero-plane lanes (the columns j with j mod S = s).
// A segment with a lane whose piece is longer than its slot is not coded here
// but appended to `list`, which seg_code_kernel then codes; a passthrough
// unit's segment is its masked bytes and sidecar, written by one coder wave.
// ctl[0]: ticket counter, ctl[1]: list length (both set before the launch).
template <int SPE, bool ESC, int PAIRS, int NPK>
__global__ void __launch_bounds__(64 * (2 + NPK) * PAIRS) __attribute__((amdgpu_waves_per_eu(4)))
seg_fast_kernel(const uint8_t* __restrict__ src, EncodeGeom g, const EncSym* __restrict__ d_enc,
                const uint32_t* __restrict__ canon, uint32_t cw, uint32_t S, uint32_t n_full, uint32_t n_last,
                FastEncParams fp,
                const uint2* __restrict__ rec, const ckr_stream_header* __restrict__ hdrs,
                const uint32_t* __restrict__ unit_size, const uint64_t* __restrict__ unit_off,
                uint8_t* __restrict__ sidecar, uint8_t* __restrict__ out, uint32_t* __restrict__ ctl,
                SegItem* __restrict__ list, uint32_t* __restrict__ err) {
    extern __shared__ uint32_t lds[];
    uint8_t* lds8 = reinterpret_cast<uint8_t*>(lds);
    constexpr uint32_t NT = 64 * (2 + NPK) * PAIRS;
    constexpr int FL = SPE == 2 ? 2 : 1;
    const uint4* tab = reinterpret_cast<const uint4*>(lds8);
    const uint32_t ctl_off = ws_ctl_offset(fp.canon_bytes);
    const uint32_t rbytes = ws_region_bytes(fp.stride0, fp.stride1);
    const uint32_t reg0 = ctl_off + PAIRS * (uint32_t)sizeof(WsPairCtl);
    const uint32_t tid = threadIdx.x;
    const uint32_t j = tid & 63;
    const uint32_t col = 4 * j;
    const uint32_t lm = live_mask32<SPE>();
    const uint32_t Kf = (uint32_t)(g.unit >> 8);  // rows of a whole unit: every lane's symbol count
    {   // table (EncSym → enc_quad), the canonical stream of Kf zero symbols (byte
        // order, at FE_CBYTES), control blocks
        const uint4* d_tab = reinterpret_cast<const uint4*>(d_enc);
        uint4* wt = reinterpret_cast<uint4*>(lds8);
        for (uint32_t k = tid; k < 256; k += NT) {
            const uint4 tv = d_tab[k];
            const EncSym e = {tv.x, tv.y, tv.z, tv.w};
            wt[k] = enc_quad(e);
        }
        const uint32_t* cs = canon + 3 * (4 + cw) + canon_index(canon, cw, Kf) * cw;
        uint32_t* cb32 = reinterpret_cast<uint32_t*>(lds8 + FE_CBYTES);
        for (uint32_t i = tid; i < fp.canon_bytes / 4; i += NT) cb32[i] = cs[i];
        uint32_t* c32 = reinterpret_cast<uint32_t*>(lds8 + ctl_off);
        for (uint32_t i = tid; i < PAIRS * (uint32_t)sizeof(WsPairCtl) / 4; i += NT) c32[i] = 0;
    }
    __syncthreads();

    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool coder = wv < 2 * PAIRS;
    const uint32_t pr = coder ? (wv >> 1) : (wv - 2 * PAIRS) / NPK;  // pair
    const uint32_t rl = wv & 1;                                       // coder: 0 byte FL, 1 byte 3
    const uint32_t pw = coder ? 0u : (wv - 2 * PAIRS) % NPK;          // packer index in the pair
    WsPairCtl& pc = *reinterpret_cast<WsPairCtl*>(lds8 + ctl_off + pr * (uint32_t)sizeof(WsPairCtl));
    // items: the n_last segments of a partial last unit (unit n_full), if there
    // is one, first (its top segment is coded row by row, the slowest item, so
    // it should not come last), then the S segments of each whole unit
    const uint32_t n_items = n_full * S + n_last;
    auto item_of = [&](uint32_t t, uint32_t& u, uint32_t& sg, uint32_t& len) {
        const bool whole = t >= n_last;
        u = whole ? (t - n_last) / S : n_full;
        sg = whole ? (t - n_last) % S : n_last - 1 - t;
        len = whole ? (uint32_t)g.unit : (uint32_t)(g.n_bytes - (uint64_t)n_full * g.unit);
    };
    // exchange words of a set (lane index li = 64 rank + column): [0, 128)
    // piece bytes, [128, 256) piece offset in the unit's output, [256, 384)
    // flags (1: longer than its slot, 2: not at its checkpoint)
    constexpr uint32_t X_LEN = 0, X_DST = 128, X_FLAG = 256;
    static_assert(NPK == 4, "four packer waves, 32 lanes' pieces each");
    static_assert(R_REC + 4 * 384 <= R_SLOTS - 516, "exchange words below the guard of the lowest slot");

    if (coder) {
        const uint32_t li = 64 * rl + j;
        const uint32_t lane = col + (rl ? 3u : (uint32_t)FL);
        for (uint32_t i = 0;; i++) {
            const uint32_t s = i & 1;
            if (i >= 2) ws_wait_ge(&pc.freed[s], i >> 1);  // set s given back
            if (rl == 0) {
                if (j == 0) pc.unit[s] = atomicAdd(&ctl[0], 1u);  // ticket
                ws_signal(&pc.tick, 1u, j);
            } else {
                ws_wait_ge(&pc.tick, i + 1);
            }
            const uint32_t t = __builtin_amdgcn_readfirstlane(ws_load(&pc.unit[s]));
            if (t >= n_items) {
                ws_signal(&pc.coded[s], 1u, j);
                break;
            }
            uint32_t u, sg, len;
            item_of(t, u, sg, len);
            const uint64_t ubase0 = (uint64_t)u * g.unit;       // the unit's first byte
            const uint64_t ubase = ubase0 + 65536ull * sg;      // the segment's first byte
            const uint32_t lo = 256 * sg;                      // the segment's rows [lo, lo + 256), clipped
            // all 256 rows of the segment full (always so in a whole unit)
            const bool full = (lo + 256) * 256 <= len;
            const uint32_t rb = reg0 + (2 * pr + s) * rbytes;
            uint32_t* xch = reinterpret_cast<uint32_t*>(lds8 + rb + R_REC);
            uint32_t e = 0, flag = 0;
            if (unit_size[u] >= len) {
                // passthrough unit: the segment's masked bytes in place, and its sidecar
                if (rl == 0) {
                    uint8_t* ud = out + unit_off[u];
                    const uint8_t* us = src + ubase0;
                    const uint32_t khi = min(lo + 256, (len + 255) / 256);
                    for (uint32_t k = lo; k < khi; k++) {
                        const uint32_t p = 256 * k + col;
                        if (p >= len) break;
                        const uint32_t nv = min(len - p, 4u);
                        uint32_t wd = 0;
                        if (nv == 4) wd = *reinterpret_cast<const uint32_t*>(us + p);
                        else for (uint32_t b = 0; b < nv; b++) wd |= (uint32_t)us[p + b] << (8 * b);
                        write_sidecar_row<SPE>(sidecar, ubase0 + p, wd, nv);
                        uint8_t* d = ud + p;
                        if (nv == 4 && (reinterpret_cast<uintptr_t>(d) & 3u) == 0) *reinterpret_cast<uint32_t*>(d) = wd & lm;
                        else
                            for (uint32_t b = 0; b < nv; b++) d[b] = (uint8_t)((wd & lm) >> (8 * b));
                    }
                }
            } else {
                uint32_t x0;
                {
                    const ckr_stream_header h = hdrs[(uint64_t)u * 256 + lane];
                    const uint2 ent = rec[((uint64_t)u * S + sg) * 128 + li];
                    const uint2 nxt = sg ? rec[((uint64_t)u * S + sg - 1) * 128 + li]
                                         : make_uint2(h.final_state, h.byte_count);
                    // the piece's place, its length and the state after it wait in
                    // the set's exchange words while the segment is coded
                    xch[X_DST + li] = h.buf_offset + h.byte_count - nxt.y;
                    xch[X_LEN + li] = nxt.y - ent.y;
                    xch[X_FLAG + li] = nxt.x;
                    x0 = ent.x;
                }
                const uint32_t sl = rl ? fp.sl1 : fp.sl0;
                if (__ballot(xch[X_LEN + li] > sl) != 0) {
                    flag = 1;  // the whole segment goes to seg_code_kernel
                } else {
                    const uint32_t endw = rl ? rb + R_SLOTS + 64 * fp.stride0 + j * fp.stride1 + fp.sl1
                                             : rb + R_SLOTS + j * fp.stride0 + fp.sl0;
                    EncLane c{x0, 0u, 0u, 0x08090A0Bu, endw - 4u};
                    EncLane c_unused = c;
                    if (full) {
                        const uint8_t* ucol = src + ubase + col;
                        if (rl == 0) enc_full_rows<SPE, ESC, true, 0, ENC_GR, ENC_TB, ENC_NBUF>(c, c_unused, ucol, sidecar, ubase, j, 256, tab, lds8);
                        else enc_full_rows<SPE, ESC, true, 1, ENC_GR, ENC_TB, ENC_NBUF>(c, c_unused, ucol, sidecar, ubase, j, 256, tab, lds8);
                    } else {
                        // the top segment of a partial last unit: rows from the top down,
                        // one at a time (as in encode_fast_kernel); the top row may be
                        // partial (bf16: lane 4j+3 has one symbol fewer)
                        const uint8_t* us = src + ubase0;
                        const uint32_t kc = len > col ? (len - col + 255) / 256 : 0u;  // rows of column j
                        const uint32_t khi = min(lo + 256, kc);
                        const uint32_t sh = rl ? 24u : 8u * FL;
                        for (int32_t k = (int32_t)khi - 1; k >= (int32_t)lo; k--) {
                            const uint32_t p = 256 * (uint32_t)k + col;
                            const uint32_t nvalid = (len - p) < 4 ? (len - p) : 4;
                            uint32_t v = 0;
                            if (nvalid == 4) v = *reinterpret_cast<const uint32_t*>(us + p);
                            else for (uint32_t b = 0; b < nvalid; b++) v |= (uint32_t)us[p + b] << (8 * b);
                            if ((uint32_t)(k & 1) == rl) write_sidecar_row<SPE>(sidecar, ubase0 + p, v, nvalid);
                            v &= lm;
                            const uint32_t sy = (v >> sh) & 255u;
                            if (rl == 0 || nvalid == 4) enc_step<ESC>(c, sy, tab[sy]);
                            if ((k & 1) == 0) enc_flush(c, lds8);
                        }
                    }
                    e = enc_finish(c, lds8, endw);
                    flag = (e == xch[X_LEN + li] && c.x == xch[X_FLAG + li]) ? 0u : 2u;
                    if (flag) e = 0;  // nothing is copied from a lane off its checkpoints
                }
            }
            xch[X_LEN + li] = e;
            xch[X_FLAG + li] = flag;
            ws_signal(&pc.coded[s], 1u, j);
        }
        return;
    }

    // packer waves
    uint32_t bar = 0;
    auto pbar_sync = [&]() {
        bar += NPK;
        ws_signal(&pc.pbar, 1u, j);
        ws_wait_ge(&pc.pbar, bar);
    };
    for (uint32_t i = 0;; i++) {
        const uint32_t s = i & 1;
        ws_wait_ge(&pc.coded[s], 2 * ((i >> 1) + 1));
        const uint32_t t = __builtin_amdgcn_readfirstlane(ws_load(&pc.unit[s]));
        if (t >= n_items) break;
        uint32_t u, sg, len;
        item_of(t, u, sg, len);
        const uint32_t rb = reg0 + (2 * pr + s) * rbytes;
        const uint32_t* xch = reinterpret_cast<const uint32_t*>(lds8 + rb + R_REC);
        const bool raw = unit_size[u] >= len;
        const uint32_t f = xch[X_FLAG + j] | xch[X_FLAG + 64 + j];
        const bool over = __ballot(f & 1u) != 0;
        const bool bad = __ballot(f & 2u) != 0;
        uint8_t* ud = out + unit_off[u];
        if (!raw && over) {
            if (pw == 0 && j == 0) {
                const uint32_t k = atomicAdd(&ctl[1], 1u);
                list[k] = SegItem{u, sg | (1u << 16)};
            }
        } else if (!raw) {
            if (bad && pw == 0 && j == 0) atomicOr(err, 1u);
            // pieces of lanes [32 pw, 32 pw + 32), in 16-byte chunks aligned in
            // memory.  First the chunks wholly inside a piece, four lanes at a time
            // (thread j: lane li0 + j / 16, chunks j mod 16, +16, ...); then the
            // piece's first and last chunks where they are partial, one per thread
            // (lane 32 pw + j / 2, its first chunk for even j, its last for odd j),
            // in byte stores.
            auto piece = [&](uint32_t li, uint32_t& e, uint8_t*& p0, int32_t& lead, uint32_t& endl) {
                e = xch[X_LEN + li];
                p0 = ud + xch[X_DST + li];
                lead = (int32_t)(reinterpret_cast<uintptr_t>(p0) & 15u);
                endl = li < 64 ? rb + R_SLOTS + li * fp.stride0 + fp.sl0
                               : rb + R_SLOTS + 64 * fp.stride0 + (li - 64) * fp.stride1 + fp.sl1;
            };
            for (uint32_t li0 = 32 * pw; li0 < 32 * pw + 32; li0 += 4) {
                uint32_t e, endl;
                uint8_t* p0;
                int32_t lead;
                piece(li0 + (j >> 4), e, p0, lead, endl);
                const uint32_t nch = e ? (uint32_t)((lead + (int32_t)e + 15) >> 4) : 0u;
                for (uint32_t ch = j & 15u; ch < nch; ch += 16) {
                    const int32_t q = 16 * (int32_t)ch - lead;  // piece offset of the chunk's first byte
                    if (q >= 0 && q + 16 <= (int32_t)e)
                        *reinterpret_cast<uint4*>(p0 + q) = lds_read16(lds8, (uint32_t)((int32_t)(endl - e) + q));
                }
            }
            {
                uint32_t e, endl;
                uint8_t* p0;
                int32_t lead;
                piece(32 * pw + (j >> 1), e, p0, lead, endl);
                const uint32_t nch = e ? (uint32_t)((lead + (int32_t)e + 15) >> 4) : 0u;
                const uint32_t ch = (j & 1u) ? nch - 1 : 0u;
                const int32_t q = 16 * (int32_t)ch - lead;
                const bool part = nch && (q < 0 || q + 16 > (int32_t)e) && !((j & 1u) && nch == 1);
                if (part) {
                    const uint4 v = lds_read16(lds8, (uint32_t)((int32_t)(endl - e) + q));
                    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int b = 0; b < 16; b++) {
                        const int32_t x = q + b;
                        if (x >= 0 && x < (int32_t)e) p0[x] = (uint8_t)(w4[b >> 2] >> (8 * (b & 3)));
                    }
                }
            }
            // the unit's zero-plane lanes (2 per column; the columns j with j mod
            // S = s): their canonical streams, one lane at a time per packer wave.
            // A partial last unit's (whose lanes have two lengths): by thread,
            // from the canonical entries in memory, the columns j with j mod
            // n_last = s.
            constexpr uint32_t ZB1 = SPE == 2 ? 1u : 2u;  // zero bytes of a column: 0 and ZB1
            if (u == n_full) {
                if (pw == 0 && j % n_last == sg) {
                    const uint32_t* cbytes = canon + 3 * (4 + cw);
                    const uint32_t kf = len >> 8, r = len & 255u;
#pragma unroll
                    for (int hz2 = 0; hz2 < 2; hz2++) {
                        const uint32_t lane = col + (hz2 ? ZB1 : 0u);
                        const ckr_stream_header hz = hdrs[(uint64_t)u * 256 + lane];
                        const uint32_t Kb = kf + ((lane < r) ? 1u : 0u);
                        seg_copy_thread(ud + hz.buf_offset, cbytes + canon_index(canon, cw, Kb) * cw, hz.byte_count);
                    }
                }
            }
            const uint32_t nz = u == n_full ? 0u : 2 * ((64 - sg + S - 1) / S);
            for (uint32_t z = pw; z < nz; z += NPK) {
                const uint32_t lane = 4 * (sg + S * (z >> 1)) + ((z & 1) ? ZB1 : 0u);
                const ckr_stream_header hz = hdrs[(uint64_t)u * 256 + lane];
                const uint32_t e = hz.byte_count <= fp.canon_bytes ? hz.byte_count : 0u;
                if (hz.byte_count > fp.canon_bytes && j == 0) atomicOr(err, 1u);
                uint8_t* p0 = ud + hz.buf_offset;
                const int32_t lead = (int32_t)(reinterpret_cast<uintptr_t>(p0) & 15u);
                const uint32_t nch = e ? (uint32_t)((lead + (int32_t)e + 15) >> 4) : 0u;
                for (uint32_t ch = j; ch < nch; ch += 64) {
                    const int32_t q = 16 * (int32_t)ch - lead;
                    const uint4 v = lds_read16(lds8, (uint32_t)((int32_t)FE_CBYTES + q));
                    if (q >= 0 && q + 16 <= (int32_t)e) {
                        *reinterpret_cast<uint4*>(p0 + q) = v;
                    } else {
                        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int b2 = 0; b2 < 16; b2++) {
                            const int32_t x = q + b2;
                            if (x >= 0 && x < (int32_t)e) p0[x] = (uint8_t)(w4[b2 >> 2] >> (8 * (b2 & 3)));
                        }
                    }
                }
            }
        }
        pbar_sync();  // every packer is done with the set
        if (pw == 0) ws_signal(&pc.freed[s], 1u, j);
    }
}

__global__ void seg_fast_reset_kernel(uint32_t* ctl) {
    if (threadIdx.x < 2) ctl[threadIdx.x] = 0;
}

uint32_t encode_seg_segments(uint64_t unit) { return seg_count(unit); }

uint64_t encode_seg_list_items(uint64_t n_units, uint64_t unit) { return n_units * seg_count(unit) + 1; }

// Coder pairs of seg_fast_kernel: 2 when they fit the LDS limit, else 0 (one
// pair per CU codes about 1.7x slower than two, and slower than
// seg_code_kernel; that happens with slots sized for the worst case, when no
// plane histograms come with the table).
static uint32_t seg_fast_pairs(const FastEncParamsHost& p, uint32_t lds_limit) {
    return ws_lds_bytes(2, p.canon_bytes, slot_stride(p.sl0), slot_stride(p.sl1)) <= lds_limit ? 2u : 0u;
}

uint32_t encode_seg_fast_lds_bytes(const FastEncParamsHost& p, uint32_t lds_limit) {
    const uint32_t pairs = seg_fast_pairs(p, lds_limit);
    return pairs ? ws_lds_bytes(pairs, p.canon_bytes, slot_stride(p.sl0), slot_stride(p.sl1)) : 0u;
}

hipError_t launch_encode_seg(const uint8_t* src, const EncodeGeom& g, const EncSym* d_enc, const uint32_t* canon,
                             uint32_t cw, bool escapes, uint2* rec, ckr_stream_header* hdrs, uint32_t* unit_size,
                             uint64_t* unit_off, uint8_t* sidecar, uint8_t* out, uint32_t* aux,
                             const FastEncParamsHost* fph, uint32_t lds_limit, uint32_t* ctl, void* list_v,
                             hipStream_t s) {
    const uint32_t S = seg_count(g.unit);
    const uint32_t g1 = (uint32_t)((g.n_units + 3) / 4);
    // segments per pass-2 item: whole units while there are units enough to
    // fill the device (>= 4096 waves), fewer otherwise
    const uint64_t G = std::max<uint64_t>(1, std::min<uint64_t>(S, g.n_units * S / 4096));
    const uint64_t items = g.n_units * ((S + G - 1) / G);
    const uint32_t g2 = (uint32_t)((items + 3) / 4);
    SegItem* list = static_cast<SegItem*>(list_v);
    // pass 2 on the fast encoder's waves: whole units of 256-row segments only
    const uint32_t pairs = (fph && (g.unit & 65535u) == 0 && ctl && list) ? seg_fast_pairs(*fph, lds_limit) : 0u;
    hipError_t e;
    int dev = 0, ncu = 0;
    if (pairs) {
        if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
        if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    }
    const bool partial = g.n_bytes % g.unit != 0;
    const uint32_t n_full = (uint32_t)(g.n_units - (partial ? 1 : 0));
    // segments of the partial last unit (rows of up to 256 bytes, 256 rows each)
    const uint64_t last_len = g.n_bytes - (g.n_units - 1) * g.unit;
    const uint32_t n_last =
        partial ? (uint32_t)((((last_len + 255) / 256) + SEG_ROWS - 1) / SEG_ROWS) : 0u;
    FastEncParams fp{};
    if (pairs) {
        fp.sl0 = fph->sl0; fp.sl1 = fph->sl1; fp.cw = fph->cw; fp.canon_bytes = fph->canon_bytes;
        fp.stride0 = slot_stride(fph->sl0); fp.stride1 = slot_stride(fph->sl1);
    }
    auto run_fast = [&](auto kern, uint32_t nthreads) -> hipError_t {
        const void* kf = reinterpret_cast<const void*>(kern);
        const uint32_t lb = ws_lds_bytes(pairs, fp.canon_bytes, fp.stride0, fp.stride1);
        hipError_t r = hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lb);
        if (r != hipSuccess) return r;
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, nthreads, lb) != hipSuccess || per_cu < 1)
            per_cu = 1;
        const uint64_t need = ((uint64_t)n_full * S + n_last + pairs - 1) / pairs;
        const uint32_t grid = (uint32_t)std::max<uint64_t>(
            1, std::min<uint64_t>(need, (uint64_t)per_cu * (uint64_t)std::max(ncu, 1)));
        CKR_LAUNCH("seg_fast_kernel", s,
                   kern<<<grid, nthreads, lb, s>>>(src, g, d_enc, canon, cw, S, n_full, n_last, fp, rec, hdrs, unit_size,
                                                   unit_off, sidecar, out, ctl, list, aux));
        return hipGetLastError();
    };
#define CKR_SEG_FAST(SPE_, ESC_) run_fast(seg_fast_kernel<SPE_, ESC_, 2, ENC_NPK>, 128u * (2 + ENC_NPK))
#define CKR_SEG(SPE_, ESC_)                                                                                         \
    do {                                                                                                            \
        CKR_LAUNCH("seg_size_kernel", s, seg_size_kernel<SPE_, ESC_><<<g1, 256, 0, s>>>(src, g, d_enc, canon, cw,    \
                                                                                        S, rec, hdrs, unit_size, aux)); \
        if ((e = hipGetLastError()) != hipSuccess) return e;                                                        \
        CKR_LAUNCH("unit_scan_kernel", s, unit_scan_kernel<<<1, 1024, 0, s>>>(unit_size, 0, g.n_units, unit_off));  \
        if ((e = hipGetLastError()) != hipSuccess) return e;                                                        \
        if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(seg_code_kernel<SPE_, ESC_, false>),             \
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)SEG_LDS)) != hipSuccess)      \
            return e;                                                                                               \
        if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(seg_code_kernel<SPE_, ESC_, true>),              \
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)SEG_LDS)) != hipSuccess)      \
            return e;                                                                                               \
        if (!pairs) {                                                                                               \
            CKR_LAUNCH("seg_code_kernel", s, seg_code_kernel<SPE_, ESC_, false><<<g2, 256, SEG_LDS, s>>>(src, g,   \
                       d_enc, canon, cw, S, (uint32_t)G, rec, hdrs, unit_size, unit_off, sidecar, out, aux,         \
                       nullptr, nullptr));                                                                          \
            return hipGetLastError();                                                                               \
        }                                                                                                           \
        CKR_LAUNCH("seg_fast_reset_kernel", s, seg_fast_reset_kernel<<<1, 64, 0, s>>>(ctl));                        \
        if ((e = hipGetLastError()) != hipSuccess) return e;                                                        \
        if ((e = CKR_SEG_FAST(SPE_, ESC_)) != hipSuccess) return e;                                                 \
        /* the listed items (usually none): a resident grid whose waves stride over the list */                     \
        const uint32_t gl = (uint32_t)std::max(ncu, 1) * 3u;                                                        \
        CKR_LAUNCH("seg_code_kernel.list", s, seg_code_kernel<SPE_, ESC_, true><<<gl, 256, SEG_LDS, s>>>(src, g,    \
                   d_enc, canon, cw, S, (uint32_t)G, rec, hdrs, unit_size, unit_off, sidecar, out, aux, list,       \
                   ctl + 1));                                                                                       \
        return hipGetLastError();                                                                                   \
    } while (0)
    if (g.spe == 2) {
        if (escapes) CKR_SEG(2, true);
        CKR_SEG(2, false);
    }
    if (escapes) CKR_SEG(1, true);
    CKR_SEG(1, false);
#undef CKR_SEG
#undef CKR_SEG_FAST
}

// ------------------------------------------------------------------ rANS decode
__device__ __forceinline__ uint32_t unit_len(const EncodeGeom& g, uint64_t ubase) {
    return (uint32_t)((g.n_bytes - ubase < g.unit) ? (g.n_bytes - ubase) : g.unit);
}

template <int SPE>
__device__ __forceinline__ uint32_t merge_sidecar_row(const uint8_t* sidecar, uint64_t pos, uint32_t dec, uint32_t nvalid) {
    if (SPE == 2) return dec | *reinterpret_cast<const uint16_t*>(sidecar + (pos >> 1));
    if (SPE == 1) {
        const uint64_t e0 = pos >> 1;
        if (nvalid >= 4) {
            const uint32_t s = *reinterpret_cast<const uint16_t*>(sidecar + e0);
            return dec | (s & 0xFFu) | ((s & 0xFF00u) << 8);
        }
        return dec | sidecar[e0];
    }
    return dec;
}

// Raw unit: masked bytes | sidecar, written by one wave (thread j: column j).
template <int SPE>
__device__ __forceinline__ void decode_raw_unit(const uint8_t* ud, uint64_t ubase, uint32_t len, uint32_t j,
                                                const uint8_t* sidecar, uint8_t* dst) {
    for (uint64_t p = 4ull * j; p < len; p += 256) {
        const uint32_t nvalid = (uint32_t)((len - p) < 4 ? (len - p) : 4);
        uint32_t v = 0;
        for (uint32_t b = 0; b < nvalid; b++) v |= (uint32_t)ud[p + b] << (8 * b);
        if (SPE > 0) v = merge_sidecar_row<SPE>(sidecar, ubase + p, v, nvalid);
        uint8_t* d = dst + ubase + p;
        if (nvalid == 4) *reinterpret_cast<uint32_t*>(d) = v;
        else for (uint32_t b = 0; b < nvalid; b++) d[b] = (uint8_t)(v >> (8 * b));
    }
}

// General decoder: any unit size, any dtype; every lane decoded from global
// memory.
struct LaneIn {
    uint32_t x;
    const uint8_t* p;
    const uint8_t* end;
};

__device__ __forceinline__ uint32_t decode_symbol(LaneIn& in, const uint32_t* tab) {
    const uint32_t slot = in.x & (M - 1u);
    const uint32_t e = tab[slot];
    const uint32_t f = ((e >> 8) & 4095u) + 1u, cum = e >> 20;
    in.x = f * (in.x >> 12) + slot - cum;
    while (in.x < L && in.p < in.end) in.x = (in.x << 8) | *in.p++;
    return e & 255u;
}

template <int SPE>
__global__ void __launch_bounds__(256) decode_kernel(const uint8_t* __restrict__ data,
                                                     const ckr_stream_header* __restrict__ hdrs,
                                                     const uint64_t* __restrict__ unit_off,
                                                     const uint32_t* __restrict__ d_dec, EncodeGeom g,
                                                     const uint8_t* __restrict__ sidecar,
                                                     uint8_t* __restrict__ dst, unsigned long long* bad) {
    __shared__ uint32_t tab[4096];
    const uint32_t j = threadIdx.x & 63;
    const uint64_t u = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    for (uint32_t i = threadIdx.x; i < 4096; i += 256) tab[i] = d_dec[i];
    __syncthreads();
    if (u >= g.n_units) return;
    const uint64_t ubase = u * g.unit;
    const uint32_t len = unit_len(g, ubase);
    const uint8_t* ud = data + unit_off[u];
    const uint64_t usize = unit_off[u + 1] - unit_off[u];
    const ckr_stream_header* uh = hdrs + u * 256;
    const uint64_t col = 4ull * j;
    if (usize == len && uh[0].byte_count == len) {
        decode_raw_unit<SPE>(ud, ubase, len, j, sidecar, dst);
        return;
    }
    LaneIn in[4];
    uint32_t nbad = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const ckr_stream_header h = uh[4 * j + b];
        in[b].x = h.final_state;
        if ((uint64_t)h.buf_offset + h.byte_count <= usize) {
            in[b].p = ud + h.buf_offset;
            in[b].end = in[b].p + h.byte_count;
        } else {  // header points outside its unit: read nothing, count the lane as bad
            in[b].p = in[b].end = ud;
            nbad++;
        }
    }
    const uint64_t K = (len > col) ? (len - col + 255) / 256 : 0;
    uint8_t* udst = dst + ubase;
    for (uint64_t k = 0; k < K; k++) {
        const uint64_t p = 256 * k + col;
        const uint32_t nvalid = (uint32_t)((len - p) < 4 ? (len - p) : 4);
        uint32_t v = 0;
        if (nvalid == 4) {
#pragma unroll
            for (int b = 0; b < 4; b++) v |= decode_symbol(in[b], tab) << (8 * b);
            if (SPE > 0) v = merge_sidecar_row<SPE>(sidecar, ubase + p, v, 4);
            *reinterpret_cast<uint32_t*>(udst + p) = v;
        } else {
#pragma unroll
            for (int b = 0; b < 4; b++)
                if ((uint32_t)b < nvalid) v |= decode_symbol(in[b], tab) << (8 * b);
            if (SPE > 0) v = merge_sidecar_row<SPE>(sidecar, ubase + p, v, nvalid);
            for (uint32_t b = 0; b < nvalid; b++) udst[p + b] = (uint8_t)(v >> (8 * b));
        }
    }
#pragma unroll
    for (int b = 0; b < 4; b++) nbad += (in[b].x != L || in[b].p != in[b].end) ? 1u : 0u;
    if (nbad) atomicAdd(bad, (unsigned long long)nbad);
}

// Fast decoder (masked planes, spe > 0; every unit of a tensor).  One block of DF_WAVES waves per CU, persistent over the units; a wave
// decodes one unit at a time, thread j taking column j, whose two live lanes
// it decodes side by side.  LDS holds the decode table, 4096 entries of
// {f | sym << 24, slot - cum} (the state update is one 24-bit multiply-add),
// and per live lane a ring with 128 bytes of its stream: two 64-byte chunks,
// chunk k of the stream (from the unit's 64-byte aligned base) in slot k & 1.
// A ring is stored dword-major: its dword r (stream bytes 4r..4r+3 modulo 128)
// is in row r, a row being 64 dwords, one per thread, so the lanes of a wave
// always read distinct banks; row 32 repeats row 0, so the two dwords around
// any byte are one ds_read2st64.  Stream bytes are taken in pairs of symbols:
// the 4 bytes at p serve both.  Rows go in groups of 8, which consume at most
// 16 bytes of a lane: when a group ends with p in chunk ch + 1 (ch: the chunk of
// p at the previous check), the lane moves on to it and fetches chunk ch + 2
// (four 16-byte loads of one 64-byte span, so each line of the stream is read
// from L2 in two pieces at most), written into the slot of chunk ch at the end
// of the next group, three groups at least before it is read.  No chunk after
// the one holding the stream's last byte is fetched: a window may take bytes
// past the end from a stale slot, but a valid stream never consumes them (a
// corrupt one fails the final state check).  The decoded
// tensor and the sidecar are streamed with non-temporal accesses so that they
// do not push the streams' lines out of L2.  Zero-plane lanes are checked
// against the canonical stream (header and bytes) and produce zeros.  A
// tensor's last unit may end in a partial row, decoded after the full rows
// with exact-size sidecar loads and byte stores.  Chunks that do not lie wholly
// inside the data buffer (the first unit of a buffer that is not 64-byte
// aligned, the units at its end, streams running past their end) are
// assembled byte by byte, with zeros outside the buffer.
static constexpr uint32_t DF_WAVES = 8;
static constexpr uint32_t DF_AHEAD = 2;  // groups of sidecar words loaded ahead of the group decoded
static constexpr uint32_t DF_CH_LOG = 6;  // chunk bytes
static constexpr uint32_t DF_CH = 1u << DF_CH_LOG;
static constexpr uint32_t DF_CQ = DF_CH / 16;  // 16-byte loads per chunk
static constexpr uint32_t DF_RING_ROWS = DF_CH / 2;  // two chunks of DF_CH / 4 dwords
// Group ends between a chunk's fetch and its write to LDS.  A lane enters
// chunk ch + 1 at a group end with p <= DF_CH (ch + 1) + 15 and takes at most 16
// bytes a group; a window reads up to 7 bytes past p.  The chunk after must be
// in LDS before any read can reach it, also in the rows after the last full
// group (at most 8 symbols, 16 bytes, no group end): 16 DF_PUT_AFTER + 21 <= DF_CH.
static constexpr uint32_t DF_PUT_AFTER = 1;
static_assert(DF_PUT_AFTER >= 1 && 16 * DF_PUT_AFTER + 21 <= DF_CH, "a chunk would be read before it is written");
static constexpr uint32_t DF_TAB_BYTES = 4096 * 4;
static constexpr uint32_t DF_RING_BYTES = (DF_RING_ROWS + 1) * 256;  // the rows + the copy of row 0
static constexpr uint32_t DF_WAVE_BYTES = 2 * DF_RING_BYTES;

// The dword at byte offset o (a multiple of 4) of the data buffer.
__device__ __forceinline__ const uint32_t* data32_at(const uint8_t* data, uint64_t o) {
    return reinterpret_cast<const uint32_t*>(data + o);
}

// One live lane of the fast decoder.
struct DfLane {
    uint32_t x;        // rANS state
    uint32_t p8;       // 8 x (position of the next stream byte, from the unit's 64-byte aligned base)
    uint32_t ch;       // chunk of p at the last check
    uint32_t last;     // chunk of the stream's last byte: no chunk after it is fetched
    uint32_t tb;       // LDS address of this lane's ring column (row 0)
    uint32_t age;      // chunk ch + 1 in flight in c[]: 0 none, else group ends since its fetch
    uint4 c[DF_CQ];
};

// Where a unit's chunks come from: chunk k is the DF_CH bytes at ua + DF_CH k; the
// chunks k_lo .. k_lo + n_in - 1 lie wholly inside the data buffer [d0, d0 + dlen).
struct DfSrc {
    const uint8_t* d0;
    uint64_t dlen;
    int64_t ua;  // the unit's 64-byte aligned base, relative to d0 (-63..)
    uint32_t k_lo, n_in;  // chunks k_lo .. k_lo + n_in - 1 lie wholly inside the buffer
};

// 16 bytes at byte offset a of the buffer, with zeros outside [0, dlen): the
// rare path of df_fetch, kept out of line.
__device__ __attribute__((noinline)) uint4 df_load16_clipped(const uint8_t* d0, uint64_t dlen, int64_t a) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t v = 0;
        for (int b = 0; b < 4; b++) {
            const int64_t o = a + 4 * i + b;
            if (o >= 0 && (uint64_t)o < dlen) v |= (uint32_t)d0[o] << (8 * b);
        }
        w[i] = v;
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Chunk k of the unit: DF_CQ 16-byte loads, or, for a chunk that is not wholly
// inside the buffer, its bytes one at a time with zeros outside.
__device__ __forceinline__ void df_fetch(const DfSrc& sr, uint32_t k, uint4 (&c)[DF_CQ]) {
    const int64_t a = sr.ua + ((int64_t)k << DF_CH_LOG);
    if (k - sr.k_lo < sr.n_in) {
        const uint4* q = reinterpret_cast<const uint4*>(sr.d0 + a);
#pragma unroll
        for (uint32_t i = 0; i < DF_CQ; i++) c[i] = q[i];
    } else {
#pragma unroll
        for (uint32_t i = 0; i < DF_CQ; i++) c[i] = df_load16_clipped(sr.d0, sr.dlen, a + 16 * i);
    }
}

// Writes chunk k into ring slot k & 1 (rows DF_CH/4 s .. DF_CH/4 s + DF_CH/4 - 1;
// slot 0 also into row DF_RING_ROWS).
__device__ __forceinline__ void df_put(uint8_t* lds8, uint32_t tb, uint32_t k, const uint4 (&c)[DF_CQ]) {
    uint32_t* w = reinterpret_cast<uint32_t*>(lds8 + tb + ((k & 1u) << (DF_CH_LOG + 6)));
#pragma unroll
    for (uint32_t i = 0; i < DF_CQ; i++) {
        w[256 * i] = c[i].x; w[256 * i + 64] = c[i].y; w[256 * i + 128] = c[i].z; w[256 * i + 192] = c[i].w;
    }
    if ((k & 1u) == 0) w[64 * DF_RING_ROWS] = c[0].x;
}

// The 4 stream bytes at p, byte p in bits 31..24.
__device__ __forceinline__ uint32_t df_window(const DfLane& d, const uint8_t* lds8) {
    const uint32_t* r = reinterpret_cast<const uint32_t*>(
        lds8 + d.tb + (__builtin_amdgcn_ubfe(d.p8, 5, DF_CH_LOG - 1) << 8));
    const uint32_t d0 = r[0], d1 = r[64];
    return __builtin_amdgcn_perm(0u, __builtin_amdgcn_alignbit(d1, d0, d.p8), 0x00010203u);
}

// One symbol (the inverse of rans_encode_kernel's step, ANSCompressor.cpp:180-202):
// x = f*(x >> 12) + slot - cum, then renormalise with 8n bits from the top of w
// (stream order), n = 0, 1, 2 for x >= 2^23, 2^15 <= x < 2^23, x < 2^15 (x >= 2^11
// here), i.e. 8n = (clz(x) - 1) & 24.  The LDS table word of a slot is
// sym << 24 | (f - 1) << 12 | (slot - cum): 4 bytes, so the table takes 16 KiB
// and an eighth wave fits (f*t = (f-1)*t + t).  Returns the table word (symbol
// in bits 31..24) and the bits consumed in sh.
__device__ __forceinline__ uint32_t df_sym(uint32_t& x, uint32_t& w, uint32_t& sh, const uint32_t* tab) {
    const uint32_t te = tab[x & (M - 1u)];
    const uint32_t t = x >> 12;
    const uint32_t xx = __umul24(__builtin_amdgcn_ubfe(te, 12, 12), t) + t + (te & 4095u);
    sh = ((uint32_t)__builtin_clz(xx) - 1u) & 24u;
    const uint64_t v = (((uint64_t)xx << 32) | w) << sh;
    x = (uint32_t)(v >> 32);
    w = (uint32_t)v;
    return te;
}

// End of a group: write the chunk fetched DF_PUT_AFTER group ends ago, then
// move on if p has reached the next chunk and fetch the one after it.  Each
// group of waiting lets the fetch's load, and the output stores issued before
// it (one in-order counter), complete while the lane decodes.
__device__ __forceinline__ void df_step(DfLane& d, uint8_t* lds8, const DfSrc& sr) {
    if (d.age == DF_PUT_AFTER) { df_put(lds8, d.tb, d.ch + 1u, d.c); d.age = 0; }
    else if (d.age) d.age++;
    const bool adv = (d.p8 >> (DF_CH_LOG + 3)) > d.ch;
    d.ch += adv ? 1u : 0u;
    if (adv && d.ch + 1u <= d.last) { df_fetch(sr, d.ch + 1u, d.c); d.age = 1; }
}

template <int SPE>
__device__ __forceinline__ uint32_t df_pack(uint32_t e0, uint32_t e1, uint32_t sw, uint32_t sel) {
    return __builtin_amdgcn_perm(__builtin_amdgcn_perm(e1, e0, SPE == 2 ? 0x07030C0Cu : 0x070C030Cu), sw, sel);
}

// The decoded tensor and the sidecar are streamed once (non-temporal).
__device__ __forceinline__ void df_store(uint32_t* p, uint32_t v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ uint32_t df_ld(const uint32_t* p) { return __builtin_nontemporal_load(p); }

// Byte selector for df_pack: o = 0 or 2, the offset of the column's sidecar
// bytes in their dword.  SPE 2: bytes {s0, s1, sym FL, sym 3}; SPE 1: {s0, sym
// FL, s1, sym 3}.
template <int SPE>
__device__ __forceinline__ uint32_t df_sel(uint32_t o) {
    return SPE == 2 ? 0x07060100u + o * 0x0101u : 0x07010500u + o * 0x00010001u;
}

// Two rows: one window read per lane, two symbols from it.
template <int SPE>
__device__ __forceinline__ void df_pair(DfLane& a, DfLane& b, const uint8_t* lds8, const uint32_t* tab, uint32_t* out,
                                        uint32_t sv0, uint32_t sv1, uint32_t sel) {
    uint32_t wa = df_window(a, lds8), wb = df_window(b, lds8);
    uint32_t ha0, ha1, hb0, hb1;
    const uint32_t a0 = df_sym(a.x, wa, ha0, tab);
    const uint32_t b0 = df_sym(b.x, wb, hb0, tab);
    df_store(out, df_pack<SPE>(a0, b0, sv0, sel));
    const uint32_t a1 = df_sym(a.x, wa, ha1, tab);
    const uint32_t b1 = df_sym(b.x, wb, hb1, tab);
    df_store(out + 64, df_pack<SPE>(a1, b1, sv1, sel));
    a.p8 += ha0 + ha1;
    b.p8 += hb0 + hb1;
}

// Eight rows (sidecar words sc), then the window step.
template <int SPE>
__device__ __forceinline__ void df_group(DfLane& a, DfLane& b, uint8_t* lds8, const uint32_t* tab, uint32_t* out,
                                         const uint32_t (&sc)[8], uint32_t sel, const DfSrc& sr) {
#pragma unroll
    for (int r = 0; r < 8; r += 2) df_pair<SPE>(a, b, lds8, tab, out + 64 * r, sc[r], sc[r + 1], sel);
    df_step(a, lds8, sr);
    df_step(b, lds8, sr);
}

__device__ __forceinline__ void df_load_sc(uint32_t (&sc)[8], const uint32_t* p) {
#pragma unroll
    for (int r = 0; r < 8; r++) sc[r] = df_ld(p + 32 * r);  // rows are 128 sidecar bytes apart
}

// A zero-plane lane against the canonical stream of its symbol count: header
// (state, count, inside the unit) and, with bytes, its bytes (they do not
// enter the output: the zero planes' output bytes are the sidecar's).  The
// bytes are compared 32 at a time, all loads of a step issued together (9
// stream dwords around the bytes, 8 canonical dwords) so that the check waits
// for memory once per step; near the ends of the data buffer, byte by byte.
__device__ __forceinline__ bool df_zero_lane_ok(const ckr_stream_header& h, const uint32_t* ce, const uint32_t* cp,
                                                uint32_t cw, const uint8_t* ud, uint32_t usize, uintptr_t d0,
                                                uintptr_t d1, bool bytes) {
    if (h.final_state != ce[1] || h.byte_count != ce[2] || (uint64_t)h.buf_offset + h.byte_count > usize) return false;
    if (!bytes) return true;
    const uint8_t* sl = ud + h.buf_offset;
    const uint32_t bc = h.byte_count;
    uint32_t diff = 0;
    for (uint32_t q0 = 0; q0 < bc; q0 += 32) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(sl) + q0, aa = a & ~(uintptr_t)3;
        const uint32_t sh = (uint32_t)(a & 3u), rem = bc - q0;
        if (aa >= d0 && aa + 36 <= d1 && (q0 >> 2) + 8 <= cw) {
            const uint32_t* bp = reinterpret_cast<const uint32_t*>(aa);
            uint32_t w[9], c[8];
#pragma unroll
            for (int k = 0; k < 9; k++) w[k] = bp[k];
#pragma unroll
            for (int k = 0; k < 8; k++) c[k] = cp[(q0 >> 2) + k];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t r = rem > 4u * k ? rem - 4u * k : 0u;  // bytes of this dword inside the stream
                const uint32_t m = r >= 4 ? ~0u : (1u << (8 * r)) - 1u;
                diff |= (__builtin_amdgcn_alignbyte(w[k + 1], w[k], sh) ^ c[k]) & m;
            }
        } else {
            const uint8_t* cb = reinterpret_cast<const uint8_t*>(cp);
            for (uint32_t q = q0; q < min(bc, q0 + 32); q++) diff |= sl[q] ^ cb[q];
        }
    }
    return diff == 0;
}

// One tensor's share of the decode: workgroup blk of nblk takes units blk *
// DF_WAVES + wave, stepping by nblk * DF_WAVES.
template <int SPE>
__device__ __forceinline__ void decode_fast_body(const uint8_t* __restrict__ data,
                                                 const ckr_stream_header* __restrict__ hdrs,
                                                 const uint64_t* __restrict__ unit_off,
                                                 const uint32_t* __restrict__ d_dec,
                                                 const uint32_t* __restrict__ canon, uint32_t cw, EncodeGeom g,
                                                 const uint8_t* __restrict__ sidecar, uint8_t* __restrict__ dst,
                                                 unsigned long long* bad, uint32_t zero_bytes, uint32_t blk,
                                                 uint32_t nblk) {
    extern __shared__ uint32_t lds[];
    uint8_t* lds8 = reinterpret_cast<uint8_t*>(lds);
    const uint32_t* tab = reinterpret_cast<const uint32_t*>(lds);
    for (uint32_t i = threadIdx.x; i < 4096; i += 64 * DF_WAVES) {
        const uint32_t e = d_dec[i];  // sym | (f - 1) << 8 | cum << 20
        lds[i] = (e & 0x000FFF00u) << 4 | (i - (e >> 20)) | (e & 255u) << 24;  // sym<<24 | (f-1)<<12 | slot-cum
    }
    __syncthreads();

    const uint32_t j = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    constexpr int FL = SPE == 2 ? 2 : 1;  // first live lane of a column
    const uint64_t data_len = unit_off[g.n_units];
    const uintptr_t d0 = reinterpret_cast<uintptr_t>(data), d1 = d0 + data_len;
    const uint32_t* cbytes = canon + 3 * (4 + cw);  // canonical streams in byte order, cw dwords each
    const uint32_t tb0 = DF_TAB_BYTES + wv * DF_WAVE_BYTES + 4 * j;
    unsigned long long nbad_total = 0;

    // the next unit's headers (this thread's four lanes) are loaded while the
    // current unit is decoded
    const uint64_t ustride = (uint64_t)nblk * DF_WAVES;
    ckr_stream_header hn[4];
    auto load_headers = [&](uint64_t v) __attribute__((always_inline)) {
        const ckr_stream_header* vh = hdrs + v * 256 + 4 * j;
#pragma unroll
        for (int b = 0; b < 4; b++) hn[b] = vh[b];
    };
    if ((uint64_t)blk * DF_WAVES + wv < g.n_units) load_headers((uint64_t)blk * DF_WAVES + wv);
    for (uint64_t u = (uint64_t)blk * DF_WAVES + wv; u < g.n_units; u += ustride) {
        ckr_stream_header uh[4];
#pragma unroll
        for (int b = 0; b < 4; b++) uh[b] = hn[b];
        if (u + ustride < g.n_units) load_headers(u + ustride);
        const uint64_t ubase = u * g.unit;
        const uint32_t len = unit_len(g, ubase);
        const uint64_t uoff = unit_off[u];
        const uint8_t* ud = data + uoff;
        const uint32_t usize = (uint32_t)(unit_off[u + 1] - uoff);
        if (usize == len && __shfl(uh[0].byte_count, 0, 64) == len) {
            decode_raw_unit<SPE>(ud, ubase, len, j, sidecar, dst);
            continue;
        }
        // chunks are read from the unit's 64-byte aligned base
        const uintptr_t ua = reinterpret_cast<uintptr_t>(ud) & ~(uintptr_t)63;
        const uint32_t g0 = (uint32_t)(reinterpret_cast<uintptr_t>(ud) - ua);
        DfSrc sr;
        sr.d0 = data;
        sr.dlen = data_len;
        sr.ua = (int64_t)ua - (int64_t)d0;
        sr.k_lo = ua >= d0 ? 0u : 1u;
        {   // chunks [k_lo, k_end) end at or before d1
            const int64_t k_end = min<int64_t>(((int64_t)d1 - (int64_t)ua) >> DF_CH_LOG, 0x40000000ll);
            sr.n_in = k_end > (int64_t)sr.k_lo ? (uint32_t)(k_end - (int64_t)sr.k_lo) : 0u;
        }
        uint32_t nbad = 0;
        DfLane da, db;
        uint32_t gea8, geb8;
        {
            auto init = [&](DfLane& d, uint32_t& ge8, int b) __attribute__((always_inline)) {
                const ckr_stream_header h = uh[b];
                const bool ok = (uint64_t)h.buf_offset + h.byte_count <= usize;
                nbad += ok ? 0u : 1u;
                const uint32_t p = g0 + (ok ? h.buf_offset : 0u);
                d.x = h.final_state;
                d.p8 = p << 3;
                const uint32_t pe = p + (ok ? h.byte_count : 0u);
                ge8 = pe << 3;
                d.ch = p >> DF_CH_LOG;
                d.last = pe > p ? (pe - 1u) >> DF_CH_LOG : d.ch;
                d.age = 0;
            };
            init(da, gea8, FL);
            init(db, geb8, 3);
            da.tb = tb0;
            db.tb = tb0 + DF_RING_BYTES;
            // the first two chunks of each stream (the second only if the stream reaches it)
            uint4 ca[DF_CQ], cb[DF_CQ];
            df_fetch(sr, da.ch, ca);
            df_fetch(sr, db.ch, cb);
            const bool a2nd = da.ch + 1u <= da.last, b2nd = db.ch + 1u <= db.last;
            if (a2nd) df_fetch(sr, da.ch + 1u, da.c);
            if (b2nd) df_fetch(sr, db.ch + 1u, db.c);
            // zero-plane lanes: header and bytes must be the canonical stream (their
            // loads wait together with the chunks above)
            const uint32_t Kz = len >> 8, rz = len & 255u;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                if (lane_is_live<SPE>(b)) continue;
                const uint32_t Kb = Kz + ((4 * j + b < rz) ? 1u : 0u);  // symbols of lane 4j+b
                const uint32_t ent = (canon[0] == Kb) ? 0u : ((canon[4 + cw] == Kb) ? 1u : 2u);
                nbad += df_zero_lane_ok(uh[b], canon + ent * (4 + cw), cbytes + (uint64_t)ent * cw, cw, ud,
                                        usize, d0, d1, zero_bytes != 0) ? 0u : 1u;
            }
            df_put(lds8, da.tb, da.ch, ca);
            df_put(lds8, db.tb, db.ch, cb);
            if (a2nd) df_put(lds8, da.tb, da.ch + 1u, da.c);
            if (b2nd) df_put(lds8, db.tb, db.ch + 1u, db.c);
        }
        const uint32_t K = len >> 8;  // full rows; a partial row K follows when len % 256 != 0
        // sidecar of row k for this column: 16 bits at (ubase + 256k + 4j) / 2, read
        // as the aligned dword around them (sidecar is 16-byte aligned, ubase a
        // multiple of 256)
        const uint32_t* sc32 = reinterpret_cast<const uint32_t*>(sidecar + (ubase >> 1) + 4 * (j >> 1));
        const uint32_t sel = df_sel<SPE>(2 * (j & 1));
        uint32_t* out32 = reinterpret_cast<uint32_t*>(dst + ubase + 4 * j);
        // rows in groups of 8 (one window step).  A group's sidecar is loaded
        // DF_AHEAD groups ahead: a load completes after every store issued before it
        // (one in-order counter), so the loads of group g + DF_AHEAD are issued
        // before group g's output stores and wait only for stores DF_AHEAD groups old.  Loads are
        // unconditional (indices clamped to the last group) so the waits stay exact.
        const uint32_t ng = K >> 3;  // full groups
        if (ng) {
            constexpr uint32_t A = DF_AHEAD;
            const uint32_t gl = ng - 1;
            uint32_t sb[A + 1][8];  // buffer q holds group gi + q
            uint32_t gi = 0;
#pragma unroll
            for (uint32_t q = 0; q < A; q++) df_load_sc(sb[q], sc32 + 256 * min(q, gl));
            for (; gi + A + 1 <= ng; gi += A + 1) {
#pragma unroll
                for (uint32_t q = 0; q <= A; q++) {
                    df_load_sc(sb[(q + A) % (A + 1)], sc32 + 256 * min(gi + q + A, gl));
                    df_group<SPE>(da, db, lds8, tab, out32 + 512 * (gi + q), sb[q], sel, sr);
                }
            }
#pragma unroll
            for (uint32_t q = 0; q < A; q++)
                if (gi + q < ng) df_group<SPE>(da, db, lds8, tab, out32 + 512 * (gi + q), sb[q], sel, sr);
        }
        // at most 7 rows left: no window step needed
        uint32_t k = 8 * ng;
        for (; k + 2 <= K; k += 2) df_pair<SPE>(da, db, lds8, tab, out32 + 64 * k, sc32[32 * k], sc32[32 * (k + 1)], sel);
        if (k < K) {
            uint32_t wa = df_window(da, lds8), wb = df_window(db, lds8);
            uint32_t ha, hb;
            const uint32_t a0 = df_sym(da.x, wa, ha, tab);
            const uint32_t b0 = df_sym(db.x, wb, hb, tab);
            out32[64 * k] = df_pack<SPE>(a0, b0, sc32[32 * k], sel);
            da.p8 += ha;
            db.p8 += hb;
        }
        // the partial top row of a tensor's last unit: r bytes, nv of them in this
        // column; a live lane takes part when its byte is among them
        const uint32_t r = len & 255u;
        if (r > 4 * j) {
            const uint32_t nv = min(r - 4 * j, 4u);
            uint32_t wa = df_window(da, lds8), wb = df_window(db, lds8);
            uint32_t ha = 0, hb = 0, v = 0;
            if (nv > (uint32_t)FL) v |= (df_sym(da.x, wa, ha, tab) >> 24) << (8 * FL);
            if (nv > 3u) v |= df_sym(db.x, wb, hb, tab) & 0xFF000000u;
            da.p8 += ha;
            db.p8 += hb;
            const uint64_t pos = ubase + 256ull * K + 4 * j;
            v = merge_sidecar_row<SPE>(sidecar, pos, v, nv);
            uint8_t* d8 = dst + pos;
            if (nv == 4) *reinterpret_cast<uint32_t*>(d8) = v;
            else for (uint32_t b = 0; b < nv; b++) d8[b] = (uint8_t)(v >> (8 * b));
        }
        nbad += (da.x != L || da.p8 != gea8) ? 1u : 0u;
        nbad += (db.x != L || db.p8 != geb8) ? 1u : 0u;
        nbad_total += nbad;
    }
    if (nbad_total) atomicAdd(bad, nbad_total);
}

template <int SPE>
__global__ void __launch_bounds__(64 * DF_WAVES) decode_fast_kernel(const uint8_t* __restrict__ data,
                                                                   const ckr_stream_header* __restrict__ hdrs,
                                                                   const uint64_t* __restrict__ unit_off,
                                                                   const uint32_t* __restrict__ d_dec,
                                                                   const uint32_t* __restrict__ canon, uint32_t cw,
                                                                   EncodeGeom g, const uint8_t* __restrict__ sidecar,
                                                                   uint8_t* __restrict__ dst, unsigned long long* bad,
                                                                   uint32_t zero_bytes) {
    decode_fast_body<SPE>(data, hdrs, unit_off, d_dec, canon, cw, g, sidecar, dst, bad, zero_bytes, blockIdx.x,
                          gridDim.x);
}

// Several tensors' decodes in one launch (ckr_decode_many on a shard of small
// tensors): one workgroup per DF_WAVES units of a job, workgroup b working for
// the last job whose first workgroup is <= b, with that job's table in its
// LDS.  One launch instead of one per tensor on four
// streams, whose launches the host could not issue as fast as the small
// decodes ran.
template <int SPE>
__global__ void __launch_bounds__(64 * DF_WAVES) decode_fast_multi_kernel(DecJobs J) {
    uint32_t k = 0;
    while (k + 1 < J.n && J.j[k + 1].blk0 <= blockIdx.x) k++;
    const DecJob& b = J.j[k];
    decode_fast_body<SPE>(b.data, b.hdrs, b.unit_off, b.dec, b.canon, b.cw, b.g, b.sidecar, b.dst, b.bad,
                          b.zero_bytes, blockIdx.x - b.blk0, b.nblk);
}

// The decode set-up of several tensors in one launch, one workgroup per job:
// its decode table from the frequency table staged in device memory
// (TableArg's norm, cum), the canonical zero-plane streams from the state
// chains, and its bad-lane counter cleared.
__global__ void __launch_bounds__(256) dec_setup_multi_kernel(DecSetupJobs J, Chains ch) {
    // 16 workgroups per job, one slot each per thread; the first also writes
    // the canonical streams and clears the bad-lane counter
    const DecSetupJob& t = J.j[blockIdx.x >> 4];
    const uint32_t part = blockIdx.x & 15u;
    __shared__ uint32_t cum[257];
    __shared__ CanonLds C;
    const uint32_t s = threadIdx.x;
    for (uint32_t i = s; i < 257; i += 256) cum[i] = t.tab->cum[i];
    CanonLoad cl{};
    if (part == 0) {
        cl = canon_load(t.tab->norm[0], t.k0, t.k1, t.k2, ch);
        if (s == 0) *t.bad = 0;
        canon_put(cl, C);
    }
    __syncthreads();
    // slot j in [cum[x], cum[x] + norm[x]) decodes to x: the largest x with cum[x] <= j
    const uint32_t j = part * 256 + s;
    uint32_t lo = 0, hi = 256;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (cum[mid] <= j) lo = mid; else hi = mid;
    }
    const uint32_t f = t.tab->norm[lo];
    if (j < cum[256] && f) t.dec[j] = lo | ((f - 1u) << 8) | (cum[lo] << 20);
    if (part == 0) canon_write(t.k0, t.k1, t.k2, t.cw, C, t.canon);
}

// ------------------------------------------------------------------ long units
// Units of masked dtypes above 1 MiB: the reference's own one-stream layout of
// a tensor (unit_bytes 0: 256 lanes of up to 2^24 symbols, coded by one block
// of 256 threads in ANSCompressor.cpp:154-216) or large units.  A lane is one
// chain of state updates from the unit's top row down
// (ANSCompressor.cpp:178-203), the only serial part of the encode.  Pass 1
// (lu_chain_kernel) follows each chain with one thread, rows fetched 64
// ahead, and records its state and the bytes emitted so far at the entry of
// every LU_SEG-row segment.  The lanes' offsets then follow from the chains'
// byte counts (unit_finalize_kernel, unit_scan_kernel), and pass 2
// (lu_code_kernel) codes every segment of every lane side by side from the
// records, storing each segment's bytes at their place in its lane's stream,
// and writes the sidecar.  A zero-plane lane codes K zeros from state L: its
// stream depends on K alone, which takes two values in a unit (the lanes
// inside the partial top row and the others), so two chains serve them all.
static constexpr uint32_t LU_SEG = 1024;  // rows per segment (a multiple of 32)
static constexpr uint32_t LU_CH = 130;    // chains per unit: 64 columns x 2 live lanes, 2 zero-plane counts

// Record slots: rec[(u * S + s) * LU_CH + c] = {state, bytes emitted so far}
// of chain c of unit u at the entry of segment s (before its top row is
// coded); c = 64 p + j for live lane p (0: byte FL, 1: byte 3) of column j,
// 128 for the zero-plane lanes of kf + 1 symbols, 129 for those of kf.
template <int SPE, bool ESC>
__global__ void __launch_bounds__(64) lu_chain_kernel(const uint8_t* __restrict__ src, EncodeGeom g,
                                                      const EncSym* __restrict__ d_enc, uint32_t S,
                                                      uint2* __restrict__ rec, ckr_stream_header* __restrict__ hdrs,
                                                      uint32_t* __restrict__ err) {
    __shared__ uint4 tab[256];
    for (uint32_t i = threadIdx.x; i < 256; i += 64) tab[i] = enc_quad(d_enc[i]);
    if (blockIdx.x == 0 && threadIdx.x == 0) *err = 0;  // pass 2 runs after this grid
    __syncthreads();
    constexpr int FL = SPE == 2 ? 2 : 1;
    const uint32_t j = threadIdx.x;
    const uint32_t role = blockIdx.x % 3;  // 0: lanes 4j + FL, 1: lanes 4j + 3, 2: the zero-plane chains
    const uint64_t u = blockIdx.x / 3;
    const uint64_t ubase = u * g.unit;
    const uint32_t len = unit_len(g, ubase);
    const uint32_t kf = len >> 8, r = len & 255u;
    uint2* ur = rec + u * (uint64_t)S * LU_CH;
    uint32_t x = L, e = 0;
    if (role == 2) {
        if (j < 2) {  // thread 0: kf + 1 symbols (kf when there is no partial row), thread 1: kf
            const uint32_t K = kf + ((j == 0 && r) ? 1u : 0u);
            const uint4 t0 = tab[0];
            uint2* cr = ur + 128 + j;
            for (int32_t s = (int32_t)((K + LU_SEG - 1) / LU_SEG) - 1; s >= 0; s--) {
                cr[(uint64_t)s * LU_CH] = make_uint2(x, e);
                const uint32_t n = min(K - (uint32_t)s * LU_SEG, LU_SEG);
                uint32_t i = 0;
                for (; i + 8 <= n; i += 8) {
#pragma unroll
                    for (int q = 0; q < 8; q++) e += seg_size_step<ESC>(x, t0);
                }
                for (; i < n; i++) e += seg_size_step<ESC>(x, t0);
            }
        }
        const uint32_t x0 = __shfl(x, 0, 64), e0 = __shfl(e, 0, 64), x1 = __shfl(x, 1, 64), e1 = __shfl(e, 1, 64);
        ckr_stream_header* uh = hdrs + u * 256 + 4 * j;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            if (lane_is_live<SPE>(b)) continue;
            const bool top = 4 * j + b < r;
            ckr_stream_header h;
            h.final_state = top ? x0 : x1;
            h.byte_count = top ? e0 : e1;
            h.buf_offset = 0;
            h.pad = 0;
            uh[b] = h;
        }
        return;
    }
    const uint32_t b = role == 0 ? FL : 3;
    const uint32_t sh = 8 * b;
    const uint32_t l = 4 * j + b;
    const uint32_t K = kf + (l < r ? 1u : 0u);
    uint2* cr = ur + 64 * role + j;
    auto record = [&](uint32_t s) { cr[(uint64_t)s * LU_CH] = make_uint2(x, e); };
    if (K) record((K - 1) / LU_SEG);
    if (K > kf) e += seg_size_step<ESC>(x, tab[src[ubase + 256ull * kf + l]]);  // the partial top row
    const uint32_t* in32 = reinterpret_cast<const uint32_t*>(src + ubase) + j;  // row k at in32[64 k]
    const uint32_t ng = kf >> 5;
    for (int32_t k = (int32_t)kf - 1; k >= (int32_t)(32 * ng); k--) {
        if ((uint32_t)(k + 1) % LU_SEG == 0) record((uint32_t)k / LU_SEG);
        e += seg_size_step<ESC>(x, tab[(in32[64 * (uint64_t)k] >> sh) & 255u]);
    }
    // groups of 32 rows from the top down, the next two groups' loads in flight
    // while one is coded; table entries read 4 rows ahead
    auto load = [&](uint32_t (&rr)[32], uint32_t gi) __attribute__((always_inline)) {
        const uint32_t* p = in32 + 64 * (32 * (uint64_t)gi + 31);
#pragma unroll
        for (int i = 0; i < 32; i++) rr[i] = p[-64 * i];
    };
    auto code = [&](const uint32_t (&rr)[32], uint32_t gi) __attribute__((always_inline)) {
        if ((32 * gi + 32) % LU_SEG == 0) record((32 * gi + 31) / LU_SEG);
        uint4 ta[2][4];
#pragma unroll
        for (int i = 0; i < 4; i++) ta[0][i] = tab[(rr[i] >> sh) & 255u];
#pragma unroll
        for (int bt = 0; bt < 8; bt++) {
            if (bt < 7) {
#pragma unroll
                for (int i = 0; i < 4; i++) ta[(bt + 1) & 1][i] = tab[(rr[4 * (bt + 1) + i] >> sh) & 255u];
            }
#pragma unroll
            for (int i = 0; i < 4; i++) e += seg_size_step<ESC>(x, ta[bt & 1][i]);
        }
    };
    if (ng) {
        uint32_t ra[32], rb[32], rc[32];
        int32_t gi = (int32_t)ng - 1;
        load(ra, (uint32_t)gi);
        if (gi >= 1) load(rb, (uint32_t)gi - 1);
        for (;;) {
            if (gi >= 2) load(rc, (uint32_t)gi - 2);
            code(ra, (uint32_t)gi);
            if (--gi < 0) break;
            if (gi >= 2) load(ra, (uint32_t)gi - 2);
            code(rb, (uint32_t)gi);
            if (--gi < 0) break;
            if (gi >= 2) load(rb, (uint32_t)gi - 2);
            code(rc, (uint32_t)gi);
            if (--gi < 0) break;
        }
    }
    ckr_stream_header h;
    h.final_state = x;
    h.byte_count = e;
    h.buf_offset = 0;
    h.pad = 0;
    hdrs[u * 256 + l] = h;
}

// Pass 2: block u * S + s codes segment s of unit u; wave b takes lanes 4j + b.
// A segment's bytes [e0, e1) of the lane's emission order lie at stream
// offsets (B - e1, B - e0] read backward (the first byte emitted is the
// stream's last): they are stored from the top down, whole aligned dwords
// inside the range and single bytes at its two ends, which share dwords with
// the neighbouring segments.  Each segment must end at the next record (state
// and count), else err is set (a bug, never expected).
template <int SPE, bool ESC>
__global__ void __launch_bounds__(256) lu_code_kernel(const uint8_t* __restrict__ src, EncodeGeom g,
                                                      const EncSym* __restrict__ d_enc, uint32_t S,
                                                      const uint2* __restrict__ rec,
                                                      const ckr_stream_header* __restrict__ hdrs,
                                                      const uint32_t* __restrict__ unit_size,
                                                      const uint64_t* __restrict__ unit_off,
                                                      uint8_t* __restrict__ sidecar, uint8_t* __restrict__ out,
                                                      uint32_t* __restrict__ err) {
    __shared__ uint4 tab[256];
    tab[threadIdx.x] = enc_quad(d_enc[threadIdx.x]);
    __syncthreads();
    constexpr int FL = SPE == 2 ? 2 : 1;
    const uint32_t j = threadIdx.x & 63, b = threadIdx.x >> 6;
    const uint64_t u = blockIdx.x / S;
    const uint32_t s = blockIdx.x % S;
    const uint64_t ubase = u * g.unit;
    const uint32_t len = unit_len(g, ubase);
    const uint32_t kf = len >> 8, r = len & 255u;
    const uint32_t k0 = s * LU_SEG, k1 = min(k0 + LU_SEG, kf + (r ? 1u : 0u));
    const ckr_stream_header* uh = hdrs + u * 256;
    uint8_t* uo = out + unit_off[u];
    const uint8_t* us = src + ubase;
    // the segment's sidecar (wave b: rows k0 + b, k0 + b + 4, ...), and, for a
    // unit stored raw, its masked bytes
    const bool raw = (uint64_t)unit_size[u] == len && uh[0].byte_count == len && uh[0].final_state == 0;
    const uint32_t lm = live_mask32<SPE>();
    for (uint32_t k = k0 + b; k < k1; k += 4) {
        const uint32_t p = 256 * k + 4 * j;
        if (p >= len) continue;
        const uint32_t nvalid = min(len - p, 4u);
        uint32_t v = 0;
        if (nvalid == 4) v = *reinterpret_cast<const uint32_t*>(us + p);
        else for (uint32_t q = 0; q < nvalid; q++) v |= (uint32_t)us[p + q] << (8 * q);
        write_sidecar_row<SPE>(sidecar, ubase + p, v, nvalid);
        if (raw) {
            v &= lm;
            for (uint32_t q = 0; q < nvalid; q++) uo[p + q] = (uint8_t)(v >> (8 * q));
        }
    }
    if (raw) return;
    const uint32_t l = 4 * j + b;
    const uint32_t kl = min(k1, kf + (l < r ? 1u : 0u));  // this lane's rows end below kl
    if (k0 >= kl) return;
    const bool live = SPE == 2 ? b >= 2 : (b & 1u) == 1u;
    const uint32_t c = live ? (b == (uint32_t)FL ? 0u : 64u) + j : (l < r ? 128u : 129u);
    const uint2 st = rec[(u * S + s) * LU_CH + c];
    const ckr_stream_header h = uh[l];
    uint32_t e1 = h.byte_count, xend = h.final_state;
    if (s) {
        const uint2 nx = rec[(u * S + s - 1) * LU_CH + c];
        e1 = nx.y;
        xend = nx.x;
    }
    uint8_t* sb = uo + h.buf_offset;
    const uintptr_t hi = reinterpret_cast<uintptr_t>(sb) + h.byte_count - st.y;
    const uintptr_t lo = reinterpret_cast<uintptr_t>(sb) + h.byte_count - e1;
    const uintptr_t blo = (lo + 3) & ~(uintptr_t)3, bhi = hi & ~(uintptr_t)3;
    uintptr_t pos = hi;
    uint32_t acc = 0;
    auto put = [&](uint32_t v) __attribute__((always_inline)) {
        pos--;
        if (pos < lo) return;  // past the segment's bytes (never expected): counted below, not stored
        if (pos >= blo && pos < bhi) {
            acc = (acc << 8) | v;
            if ((pos & 3u) == 0) *reinterpret_cast<uint32_t*>(pos) = acc;
        } else {
            *reinterpret_cast<uint8_t*>(pos) = (uint8_t)v;
        }
    };
    uint32_t x = st.x;
    const uint32_t sh = 8 * b;
    for (int32_t k = (int32_t)kl - 1; k >= (int32_t)k0; k--) {
        uint32_t sym = 0;
        if (live) sym = (uint32_t)k < kf ? (*reinterpret_cast<const uint32_t*>(us + 256ull * k + 4 * j) >> sh) & 255u
                                         : us[256ull * k + l];
        const uint4 t = tab[sym];
        const uint32_t f8 = t.w;
        if (ESC && f8 == 0u) {  // raw-byte escape (ANSCompressor.cpp:185-192)
            put(sym);
            continue;
        }
        const uint32_t n = ((x >> 24) >= f8) ? 2u : (((x >> 16) >= f8) ? 1u : 0u);
        if (n >= 1) put(x & 255u);
        if (n == 2) put((x >> 8) & 255u);
        const uint32_t xr = x >> (8 * n);
        const uint32_t q = __umulhi(xr, t.x) >> (t.y >> 24);
        x = xr + t.z + __umul24(q, t.y);
    }
    if (hi - pos != (uintptr_t)(e1 - st.y) || x != xend) atomicOr(err, 1u);
}

uint32_t encode_long_segments(uint64_t unit) { return (uint32_t)(((unit + 255) / 256 + LU_SEG - 1) / LU_SEG); }
uint64_t encode_long_rec_bytes(uint64_t n_units, uint64_t unit) {
    return n_units * (uint64_t)encode_long_segments(unit) * LU_CH * sizeof(uint2);
}

template <int SPE, bool ESC>
static hipError_t encode_long_t(const uint8_t* src, const EncodeGeom& g, const EncSym* d_enc, uint2* rec,
                                ckr_stream_header* hdrs, uint32_t* unit_size, uint64_t* unit_off, uint8_t* sidecar,
                                uint8_t* out, uint32_t* err, hipStream_t s) {
    const uint32_t S = encode_long_segments(g.unit);
    CKR_LAUNCH("lu_chain_kernel", s, lu_chain_kernel<SPE, ESC><<<(uint32_t)(3 * g.n_units), 64, 0, s>>>(src, g, d_enc, S, rec, hdrs, err));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    CKR_LAUNCH("unit_finalize_kernel", s, unit_finalize_kernel<<<(uint32_t)g.n_units, 256, 0, s>>>(g, 0, hdrs, unit_size, nullptr));
    if ((e = hipGetLastError()) != hipSuccess) return e;
    CKR_LAUNCH("unit_scan_kernel", s, unit_scan_kernel<<<1, 1024, 0, s>>>(unit_size, 0, g.n_units, unit_off));
    if ((e = hipGetLastError()) != hipSuccess) return e;
    CKR_LAUNCH("lu_code_kernel", s, lu_code_kernel<SPE, ESC><<<(uint32_t)(g.n_units * S), 256, 0, s>>>(src, g, d_enc, S, rec, hdrs, unit_size, unit_off, sidecar, out, err));
    return hipGetLastError();
}

hipError_t launch_encode_long(const uint8_t* src, const EncodeGeom& g, const EncSym* d_enc, bool escapes, uint2* rec,
                              ckr_stream_header* hdrs, uint32_t* unit_size, uint64_t* unit_off, uint8_t* sidecar,
                              uint8_t* out, uint32_t* err, hipStream_t s) {
    if (g.n_units == 0) return hipSuccess;
    if (g.spe == 2)
        return escapes ? encode_long_t<2, true>(src, g, d_enc, rec, hdrs, unit_size, unit_off, sidecar, out, err, s)
                       : encode_long_t<2, false>(src, g, d_enc, rec, hdrs, unit_size, unit_off, sidecar, out, err, s);
    if (g.spe == 1)
        return escapes ? encode_long_t<1, true>(src, g, d_enc, rec, hdrs, unit_size, unit_off, sidecar, out, err, s)
                       : encode_long_t<1, false>(src, g, d_enc, rec, hdrs, unit_size, unit_off, sidecar, out, err, s);
    return hipErrorInvalidValue;
}

// Decoder of long units: each lane is one chain from its stream's start, so a
// unit takes one block of four waves, wave b decoding lanes 4j + b, one chain
// per thread (two chains interleaved in one thread took 1.8x as long: their
// table lookups end up serialised).  The zero-plane lanes must give zeros and
// end where their streams end.  Stream bytes go through the fast decoder's LDS
// rings (df_*), each lane's chunks counted from its own stream's 64-byte
// aligned start (so positions, in bits, stay below 2^29 for a lane of 2^24
// symbols).  The unit's other LU_RAW_BLOCKS blocks copy it when it is stored
// raw.
static constexpr uint32_t LU_RAW_BLOCKS = 64;

__device__ __forceinline__ void lu_lane_init(DfLane& d, DfSrc& sr, uint32_t& ge8, const ckr_stream_header& h,
                                             const uint8_t* data, uint64_t data_len, const uint8_t* ud,
                                             uint64_t usize, uint32_t& nbad) {
    const bool ok = (uint64_t)h.buf_offset + h.byte_count <= usize;
    nbad += ok ? 0u : 1u;
    const uint8_t* sp = ud + (ok ? h.buf_offset : 0u);
    const uintptr_t ua = reinterpret_cast<uintptr_t>(sp) & ~(uintptr_t)63;
    const uintptr_t d0 = reinterpret_cast<uintptr_t>(data), d1 = d0 + data_len;
    const uint32_t g0 = (uint32_t)(reinterpret_cast<uintptr_t>(sp) - ua);
    sr.d0 = data;
    sr.dlen = data_len;
    sr.ua = (int64_t)ua - (int64_t)d0;
    sr.k_lo = ua >= d0 ? 0u : 1u;
    const int64_t k_end = min<int64_t>(((int64_t)d1 - (int64_t)ua) >> DF_CH_LOG, 0x40000000ll);
    sr.n_in = k_end > (int64_t)sr.k_lo ? (uint32_t)(k_end - (int64_t)sr.k_lo) : 0u;
    d.x = h.final_state;
    d.p8 = g0 << 3;
    const uint32_t pe = g0 + (ok ? h.byte_count : 0u);
    ge8 = pe << 3;
    d.ch = 0;
    d.last = pe > g0 ? (pe - 1u) >> DF_CH_LOG : 0u;
    d.age = 0;
}

// One lane per thread: wave b of a unit's block decodes lanes 4j + b of every
// column and stores byte b of each row (a live lane its symbols, a zero-plane
// lane, which must give zeros, the sidecar's byte, loaded LU_AHEAD groups of 8
// rows ahead).
static constexpr uint32_t LU_AHEAD = 2;

template <int SPE, int B>
__device__ __forceinline__ uint32_t lu_decode_lane(const uint8_t* data, uint64_t data_len,
                                                   const ckr_stream_header* uh, const uint8_t* ud, uint64_t usize,
                                                   uint32_t len, uint64_t ubase, const uint32_t* tab, uint8_t* lds8,
                                                   uint32_t tb, const uint8_t* sidecar, uint8_t* dst, uint32_t j) {
    constexpr bool LIVE = lane_is_live<SPE>(B);
    uint32_t nbad = 0, z = 0;
    DfLane d;
    DfSrc sr;
    uint32_t ge8;
    lu_lane_init(d, sr, ge8, uh[4 * j + B], data, data_len, ud, usize, nbad);
    d.tb = tb;
    {
        uint4 c0[DF_CQ];
        df_fetch(sr, 0, c0);
        const bool second = d.last >= 1u;
        if (second) df_fetch(sr, 1, d.c);
        df_put(lds8, d.tb, 0, c0);
        if (second) df_put(lds8, d.tb, 1, d.c);
    }
    const uint32_t K = len >> 8;  // full rows; a partial row K follows when len % 256 != 0
    uint8_t* o8 = dst + ubase + 4 * j + B;  // row k at o8[256 k]
    // the zero planes' output bytes are the sidecar's: fp32 bytes 0, 1 of the
    // element; bf16 byte 0 of each of the column's two elements
    const uint8_t* s8 = sidecar + ((ubase + 4 * j) >> 1) + (SPE == 2 ? B : B / 2);  // row k at s8[128 k]
    auto pair = [&](uint32_t k, uint32_t sv0, uint32_t sv1) __attribute__((always_inline)) {
        uint32_t w = df_window(d, lds8), h0, h1;
        const uint32_t t0 = df_sym(d.x, w, h0, tab);
        const uint32_t t1 = df_sym(d.x, w, h1, tab);
        d.p8 += h0 + h1;
        if (LIVE) {
            o8[256ull * k] = (uint8_t)(t0 >> 24);
            o8[256ull * (k + 1)] = (uint8_t)(t1 >> 24);
        } else {
            z |= t0 | t1;
            o8[256ull * k] = (uint8_t)sv0;
            o8[256ull * (k + 1)] = (uint8_t)sv1;
        }
    };
    const uint32_t ng = K >> 3;
    if (ng) {
        const uint32_t gl = ng - 1;
        uint32_t sb[LU_AHEAD + 1][8];
        auto load = [&](uint32_t (&v)[8], uint32_t g) __attribute__((always_inline)) {
            if (!LIVE) {
#pragma unroll
                for (int r = 0; r < 8; r++) v[r] = s8[128ull * (8 * g + r)];
            }
        };
#pragma unroll
        for (uint32_t q = 0; q < LU_AHEAD; q++) load(sb[q], min(q, gl));
        uint32_t gi = 0;
        for (; gi + LU_AHEAD + 1 <= ng; gi += LU_AHEAD + 1) {
#pragma unroll
            for (uint32_t q = 0; q <= LU_AHEAD; q++) {
                load(sb[(q + LU_AHEAD) % (LU_AHEAD + 1)], min(gi + q + LU_AHEAD, gl));
#pragma unroll
                for (int r = 0; r < 8; r += 2) pair(8 * (gi + q) + r, sb[q][r], sb[q][r + 1]);
                df_step(d, lds8, sr);
            }
        }
#pragma unroll
        for (uint32_t q = 0; q < LU_AHEAD; q++) {
            if (gi + q < ng) {
#pragma unroll
                for (int r = 0; r < 8; r += 2) pair(8 * (gi + q) + r, sb[q][r], sb[q][r + 1]);
                df_step(d, lds8, sr);
            }
        }
    }
    uint32_t k = 8 * ng;
    for (; k + 2 <= K; k += 2) pair(k, LIVE ? 0u : s8[128ull * k], LIVE ? 0u : s8[128ull * (k + 1)]);
    const bool top = 4 * j + B < (len & 255u);  // this lane holds a byte of the partial row K
    if (k < K || top) {
        uint32_t w = df_window(d, lds8), h0 = 0, h1 = 0;
        if (k < K) {
            const uint32_t t0 = df_sym(d.x, w, h0, tab);
            if (LIVE) o8[256ull * k] = (uint8_t)(t0 >> 24);
            else { z |= t0; o8[256ull * k] = s8[128ull * k]; }
            k++;
        }
        if (top) {
            const uint32_t t1 = df_sym(d.x, w, h1, tab);
            if (LIVE) o8[256ull * K] = (uint8_t)(t1 >> 24);
            else { z |= t1; o8[256ull * K] = s8[128ull * K]; }
        }
        d.p8 += h0 + h1;
    }
    // bad: not ending at state L with every byte consumed, or, in a zero
    // plane, a nonzero symbol
    nbad += (d.x != L || d.p8 != ge8 || (!LIVE && (z >> 24))) ? 1u : 0u;
    return nbad;
}

template <int SPE>
__global__ void __launch_bounds__(256) decode_long_kernel(const uint8_t* __restrict__ data,
                                                          const ckr_stream_header* __restrict__ hdrs,
                                                          const uint64_t* __restrict__ unit_off,
                                                          const uint32_t* __restrict__ d_dec, EncodeGeom g,
                                                          const uint8_t* __restrict__ sidecar,
                                                          uint8_t* __restrict__ dst, unsigned long long* bad) {
    extern __shared__ uint32_t lds[];
    const uint64_t u = blockIdx.x;
    const uint32_t j = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint64_t ubase = u * g.unit;
    const uint32_t len = unit_len(g, ubase);
    const uint64_t uoff = unit_off[u];
    const uint8_t* ud = data + uoff;
    const uint64_t usize = unit_off[u + 1] - uoff;
    const ckr_stream_header* uh = hdrs + u * 256;
    const bool raw = usize == len && uh[0].byte_count == len;
    if (blockIdx.y) {  // a raw unit: masked bytes | sidecar, rows shared by the blocks' waves
        if (!raw) return;
        const uint32_t W = 4 * LU_RAW_BLOCKS;
        for (uint32_t k = (blockIdx.y - 1) * 4 + wv; 256ull * k < len; k += W) {
            const uint32_t p = 256 * k + 4 * j;
            if (p >= len) continue;
            const uint32_t nvalid = min(len - p, 4u);
            uint32_t v = 0;
            for (uint32_t q = 0; q < nvalid; q++) v |= (uint32_t)ud[p + q] << (8 * q);
            v = merge_sidecar_row<SPE>(sidecar, ubase + p, v, nvalid);
            uint8_t* dd = dst + ubase + p;
            if (nvalid == 4) *reinterpret_cast<uint32_t*>(dd) = v;
            else for (uint32_t q = 0; q < nvalid; q++) dd[q] = (uint8_t)(v >> (8 * q));
        }
        return;
    }
    if (raw) return;
    uint8_t* lds8 = reinterpret_cast<uint8_t*>(lds);
    for (uint32_t i = threadIdx.x; i < 4096; i += 256) {
        const uint32_t e = d_dec[i];  // sym | (f - 1) << 8 | cum << 20
        lds[i] = (e & 0x000FFF00u) << 4 | (i - (e >> 20)) | (e & 255u) << 24;  // sym<<24 | (f-1)<<12 | slot-cum
    }
    __syncthreads();
    const uint64_t data_len = unit_off[g.n_units];
    const uint32_t tb = DF_TAB_BYTES + wv * DF_RING_BYTES + 4 * j;
    uint32_t nbad;
    switch (wv) {
        case 0: nbad = lu_decode_lane<SPE, 0>(data, data_len, uh, ud, usize, len, ubase, lds, lds8, tb, sidecar, dst, j); break;
        case 1: nbad = lu_decode_lane<SPE, 1>(data, data_len, uh, ud, usize, len, ubase, lds, lds8, tb, sidecar, dst, j); break;
        case 2: nbad = lu_decode_lane<SPE, 2>(data, data_len, uh, ud, usize, len, ubase, lds, lds8, tb, sidecar, dst, j); break;
        default: nbad = lu_decode_lane<SPE, 3>(data, data_len, uh, ud, usize, len, ubase, lds, lds8, tb, sidecar, dst, j); break;
    }
    if (nbad) atomicAdd(bad, (unsigned long long)nbad);
}

hipError_t launch_decode_long(const uint8_t* data, const ckr_stream_header* hdrs, const uint64_t* unit_off,
                              const uint32_t* d_dec, const EncodeGeom& g, const uint8_t* sidecar, uint8_t* dst,
                              unsigned long long* bad, hipStream_t s) {
    if (g.n_units == 0) return hipSuccess;
    if (g.spe != 1 && g.spe != 2) return hipErrorInvalidValue;
    const uint32_t lb = DF_TAB_BYTES + 4 * DF_RING_BYTES;
    const dim3 grid((uint32_t)g.n_units, 1 + LU_RAW_BLOCKS);
    if (g.spe == 2) CKR_LAUNCH("decode_long_kernel", s, decode_long_kernel<2><<<grid, 256, lb, s>>>(data, hdrs, unit_off, d_dec, g, sidecar, dst, bad));
    else CKR_LAUNCH("decode_long_kernel", s, decode_long_kernel<1><<<grid, 256, lb, s>>>(data, hdrs, unit_off, d_dec, g, sidecar, dst, bad));
    return hipGetLastError();
}

hipError_t launch_build_enc_table(const TableArg& t, EncSym* d_enc, hipStream_t s) {
    CKR_LAUNCH("build_enc_table_kernel", s, build_enc_table_kernel<<<1, 256, 0, s>>>(t, d_enc));
    return hipGetLastError();
}
hipError_t launch_build_enc_table_reset(const TableArg& t, EncSym* d_enc, uint64_t* status, uint64_t n_units,
                                        uint32_t* ctl, hipStream_t s) {
    const uint64_t nst = encode_fast_status_words(n_units);  // unit words, block words, block counts
    const uint32_t grid = (uint32_t)std::max<uint64_t>(1, (nst + 255) / 256);
    CKR_LAUNCH("build_enc_table_reset_kernel", s,
               build_enc_table_reset_kernel<<<grid, 256, 0, s>>>(t, d_enc, status, nst, ctl));
    return hipGetLastError();
}
hipError_t launch_tables(const uint32_t* hists, uint64_t n, int ensure_full, uint32_t* rows, hipStream_t s) {
    for (uint64_t b0 = 0; b0 < n; b0 += 1u << 30) {
        const uint32_t nb = (uint32_t)std::min<uint64_t>(n - b0, 1u << 30);
        CKR_LAUNCH("tables_kernel", s, tables_kernel<<<nb, 256, 0, s>>>(hists + b0 * 256, ensure_full, rows + b0 * 258));
    }
    return hipGetLastError();
}
hipError_t launch_canon_chains(void* chains, hipStream_t s) {
    uint8_t* p = static_cast<uint8_t*>(chains);
    auto* cx = reinterpret_cast<uint32_t*>(p);
    auto* cn = reinterpret_cast<uint16_t*>(p + 4ull * (kChainSteps + 1) * kChainRows);
    auto* cb = p + 6ull * (kChainSteps + 1) * kChainRows;
    CKR_LAUNCH("canon_chain_kernel", s, canon_chain_kernel<<<(kChainRows + 255) / 256, 256, 0, s>>>(cx, cn, cb));
    return hipGetLastError();
}
static Chains chains_of(const void* chains) {
    const uint8_t* p = static_cast<const uint8_t*>(chains);
    return Chains{reinterpret_cast<const uint32_t*>(p),
                  reinterpret_cast<const uint16_t*>(p + 4ull * (kChainSteps + 1) * kChainRows),
                  p + 6ull * (kChainSteps + 1) * kChainRows};
}
// A value no earlier launch of this process used, and unlikely to be left in
// memory by another process.
static uint64_t next_epoch() {
    static std::atomic<uint64_t> next{0x5a17c0de00000000ull ^ ((uint64_t)reinterpret_cast<uintptr_t>(&next) << 8)};
    return next.fetch_add(1, std::memory_order_relaxed) + 1;
}
hipError_t launch_hist_table(const HistSrc* srcs, uint32_t* const* hists, const TableEncJob* jobs, uint32_t n,
                             const void* chains, uint64_t* epochs, hipStream_t s) {
    for (uint32_t j0 = 0; j0 < n; j0 += kMaxHistJobs) {
        const uint32_t m = std::min<uint32_t>(kMaxHistJobs, n - j0);
        HistTableJobs J{};
        J.n = m;
        J.epoch = next_epoch();
        HistJob hj[kMaxHistJobs];
        for (uint32_t k = 0; k < m; k++)
            if (srcs[j0 + k].spe != 1 && srcs[j0 + k].spe != 2) return hipErrorInvalidValue;
        const uint32_t nb = hist_shares(srcs + j0, m, hj, hists + j0);
        for (uint32_t k = 0; k < m; k++) {
            J.j[k].h = hj[k];
            J.j[k].t = jobs[j0 + k];
        }
        for (uint32_t k = 0; k < m; k++) epochs[j0 + k] = J.epoch;
        CKR_LAUNCH("hist_table_kernel", s, hist_table_kernel<<<nb, 256, 0, s>>>(J, chains_of(chains)));
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
// The largest slot (bytes, a multiple of 4, at most 2K + 8) whose two-pair
// layout fits lds_cap.
uint32_t encode_fast_max_slot(uint32_t canon_bytes, uint32_t K, uint32_t lds_cap) {
    uint32_t sl = (2 * K + 8 + 3) & ~3u;
    while (sl > 8 && ws_lds_bytes(2, canon_bytes, slot_stride(sl), slot_stride(sl)) > lds_cap) sl -= 4;
    return ws_lds_bytes(2, canon_bytes, slot_stride(sl), slot_stride(sl)) <= lds_cap ? sl : 0u;
}
hipError_t launch_build_dec_table(const TableArg& t, uint32_t* d_dec, unsigned long long* bad, hipStream_t s) {
    CKR_LAUNCH("build_dec_table_kernel", s, build_dec_table_kernel<<<16, 256, 0, s>>>(t, d_dec, bad));
    return hipGetLastError();
}

uint32_t decode_fast_lds_bytes() { return DF_TAB_BYTES + DF_WAVES * DF_WAVE_BYTES; }

hipError_t launch_dec_setup_multi(const DecSetupJob* jobs, uint32_t n, const void* chains, hipStream_t s) {
    for (uint32_t j0 = 0; j0 < n; j0 += kMaxDecJobs) {
        DecSetupJobs J{};
        J.n = std::min<uint32_t>(kMaxDecJobs, n - j0);
        for (uint32_t k = 0; k < J.n; k++) J.j[k] = jobs[j0 + k];
        CKR_LAUNCH("dec_setup_multi_kernel", s, dec_setup_multi_kernel<<<16 * J.n, 256, 0, s>>>(J, chains_of(chains)));
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
hipError_t launch_decode_fast_multi(DecJob* jobs, uint32_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (n > kMaxDecJobs) return hipErrorInvalidValue;
    const int spe = jobs[0].g.spe;
    for (uint32_t i = 0; i < n; i++)
        if (jobs[i].g.spe != spe || (spe != 1 && spe != 2)) return hipErrorInvalidValue;
    const uint32_t lb = decode_fast_lds_bytes();
    int per_cu = 0;
    auto kern = spe == 2 ? decode_fast_multi_kernel<2> : decode_fast_multi_kernel<1>;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lb) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 64 * DF_WAVES, lb) != hipSuccess || per_cu < 1) {
        (void)hipGetLastError();
        return hipErrorInvalidValue;
    }
    // one workgroup per DF_WAVES units of a job (a unit per wave): more than
    // fit at once, so that the dispatcher hands the next workgroup to each CU
    // a finished one leaves (fixed shares of the resident workgroups left every
    // job several rounds, the last of them partly idle)
    DecJobs J{};
    J.n = n;
    uint64_t nb = 0;
    for (uint32_t i = 0; i < n; i++) {
        DecJob& b = jobs[i];
        b.nblk = (uint32_t)std::max<uint64_t>(1, (b.g.n_units + DF_WAVES - 1) / DF_WAVES);
        b.blk0 = (uint32_t)nb;
        nb += b.nblk;
        J.j[i] = b;
    }
    if (nb > 0x7fffffffu) return hipErrorInvalidValue;
    CKR_LAUNCH("decode_fast_kernel", s, kern<<<(uint32_t)nb, 64 * DF_WAVES, lb, s>>>(J));
    return hipGetLastError();
}
hipError_t launch_decode(const uint8_t* data, const ckr_stream_header* hdrs, const uint64_t* unit_off,
                         const uint32_t* d_dec, const EncodeGeom& g, const uint8_t* sidecar, uint8_t* dst,
                         unsigned long long* bad, const uint32_t* canon, uint32_t cw, hipStream_t s, bool zero_bytes) {
    const uint32_t grid = (uint32_t)((g.n_units + 3) / 4);
    if (grid == 0) return hipSuccess;
    hipError_t e;
    bool fast_ran = false;
    if (canon && g.spe > 0) {  // fast path
        const uint32_t lb = decode_fast_lds_bytes();
        int dev = 0, ncu = 0;
        if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
        if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
        auto fast = [&](auto kern) -> hipError_t {
            int per_cu = 0;
            if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lb) != hipSuccess ||
                hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 64 * DF_WAVES, lb) != hipSuccess || per_cu < 1) {
                (void)hipGetLastError();
                return hipSuccess;  // LDS too small on this device: the general kernel takes every unit
            }
            // persistent: the blocks that fit at once, never more than needed
            const uint64_t need = (g.n_units + DF_WAVES - 1) / DF_WAVES;
            const uint32_t fg = (uint32_t)std::min<uint64_t>(need, (uint64_t)per_cu * (uint64_t)std::max(ncu, 1));
            CKR_LAUNCH("decode_fast_kernel", s, kern<<<fg, 64 * DF_WAVES, lb, s>>>(data, hdrs, unit_off, d_dec, canon, cw, g, sidecar, dst, bad, zero_bytes ? 1u : 0u));
            fast_ran = true;
            return hipGetLastError();
        };
        if ((e = (g.spe == 2 ? fast(decode_fast_kernel<2>) : fast(decode_fast_kernel<1>))) != hipSuccess) return e;
        if (fast_ran) return hipSuccess;  // the fast kernel decodes every unit
    }
    if (g.spe == 2) CKR_LAUNCH("decode_kernel", s, decode_kernel<2><<<grid, 256, 0, s>>>(data, hdrs, unit_off, d_dec, g, sidecar, dst, bad));
    else if (g.spe == 1) CKR_LAUNCH("decode_kernel", s, decode_kernel<1><<<grid, 256, 0, s>>>(data, hdrs, unit_off, d_dec, g, sidecar, dst, bad));
    else CKR_LAUNCH("decode_kernel", s, decode_kernel<0><<<grid, 256, 0, s>>>(data, hdrs, unit_off, d_dec, g, sidecar, dst, bad));
    return hipGetLastError();
}

}  // namespace ckr
