// checkers_amd/csrc/ckr_repair.hip — tensor-group prefix-mask repair (Re-Pair
// over masked words) on the GPU.
//
// Reference: src/tensor_group_prefix_mask_repair.cpp — build_masked_sequence
// (:328-353), find_best_pair (:376-405), apply_rule (:407-426),
// build_shared_grammar (:428-457), apply_existing_grammar (:459-467).
//
// Layout.  Each masked word (word with its low k mantissa bits cleared) is
// replaced by a dense u32 id, its rank in the tensor's alphabet; rule r gets
// id A0 + r.  sym[id] keeps the reference's 64-bit symbol (the masked word, or
// 2^63 + r) for the tie-break hash.  The sequence lives in two u32 buffers
// that the rounds ping-pong between.
//
// One round (all on the device, no host synchronisation):
//   pair_pass<COUNT>   every adjacent pair counted (first round, or when the
//                      table is to be rebuilt): per-workgroup LDS cache of
//                      2048 pairs in front of a global open-addressing table;
//                      later rounds keep the counts up to date instead: the
//                      replacement subtracts the pairs it destroys (those with
//                      a replaced token) and pair_pass<INC> adds the new
//                      sequence's pairs holding the new symbol, the only new
//                      pairs (a pair of two kept tokens was a pair before);
//   sel_max/sel_cand   largest count and the number of pairs holding it;
//   tie_*              only if several pairs hold it: the pair std::unordered_map
//                      would visit first.  libstdc++ keeps one singly linked
//                      list; a node for an empty bucket goes to the list head,
//                      a node for a used bucket goes to the front of that
//                      bucket's run.  With reserve(size) no rehash happens, so
//                      the visit order is: buckets by decreasing time of their
//                      first insertion, and within a bucket pairs by decreasing
//                      time of insertion.  Insertion time is the position of a
//                      pair's first occurrence.  The winner maximises
//                      (first occurrence of any pair in its bucket, its own
//                      first occurrence); the bucket is hash % P with P the
//                      bucket count of reserve(size), taken from libstdc++ by
//                      the host;
//   round_commit       record the rule (or stop: best count < 2) and decide
//                      whether the next round recounts (table above 3/4 full
//                      once the new pairs are in);
//   rep_*              greedy left-to-right replacement as a scan: the state
//                      "previous token started a replacement" is a function of
//                      the state entering a segment, so segments compose;
//   tab_clear/round_end reset the touched table slots (recount only) and advance.
#include "ckr_internal.h"

namespace ckr {
namespace {

constexpr uint64_t EMPTY_KEY = ~0ull;
constexpr uint32_t NONE = 0xFFFFFFFFu;
constexpr int RT = 256;          // threads per workgroup
constexpr int CACHE = 2048;      // LDS pair cache entries
constexpr int CACHE_PROBES = 8;
constexpr int DCACHE = 1024;     // LDS cache of the pairs a replacement workgroup subtracts
constexpr int SEG = 16;          // tokens per thread in the replace pass
constexpr int BLK = RT * SEG;    // tokens per replace block
constexpr int SCAN_T = 1024;     // threads of the single-workgroup scans
constexpr uint32_t PAIR_CHUNK = 8192;  // least pairs per pair_pass workgroup
constexpr uint32_t PAIR_BLOCKS_PER_CU = 4;  // pair_pass workgroups per CU at most, larger chunks above
constexpr int PAIR_UNROLL = 4;   // pairs loaded together per pair_pass thread
constexpr uint32_t OCC_BLK = 4096;

// MurmurHash3 fmix64 / fmix32 finalizers (public domain): table slot hashes.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x ^= x >> 33; x *= 0xff51afd7ed558ccdull; x ^= x >> 33; x *= 0xc4ceb9fe1a85ec53ull; x ^= x >> 33;
    return x;
}
__device__ __forceinline__ uint32_t mix32(uint32_t x) {
    x ^= x >> 16; x *= 0x85ebca6bu; x ^= x >> 13; x *= 0xc2b2ae35u; x ^= x >> 16;
    return x;
}

// PairKeyHash of the reference (tensor_group_prefix_mask_repair.cpp:366-374)
// with std::hash<uint64_t> the identity.
__device__ __forceinline__ uint64_t ref_pair_hash(uint64_t l, uint64_t r) {
    return l ^ (r + 0x9e3779b97f4a7c15ull + (l << 6) + (l >> 2));
}

__device__ __forceinline__ uint64_t ld_relaxed(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int ES>
__device__ __forceinline__ uint32_t load_word(const uint8_t* w, uint64_t i) {
    if constexpr (ES == 2) return reinterpret_cast<const uint16_t*>(w)[i];
    else return reinterpret_cast<const uint32_t*>(w)[i];
}

struct PairTab {
    uint64_t* key;
    uint32_t* cnt;
    uint32_t* first;
    uint32_t* touched;
    uint64_t mask;  // capacity - 1 (power of two)
};

// ------------------------------------------------------------------ block helpers
__device__ uint32_t block_reduce_max(uint32_t v, uint32_t* sh) {
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o));
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    uint32_t r = 0;
    for (int i = 0; i < nw; i++) r = max(r, sh[i]);
    return r;
}

// Exclusive scan of u32 over the block (blockDim.x <= 1024); returns the
// exclusive prefix, *total the sum.
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t* sh, uint32_t* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    uint32_t x = v;
    for (int o = 1; o < 64; o <<= 1) {
        uint32_t y = (uint32_t)__shfl_up((int)x, o);
        if (lane >= o) x += y;
    }
    __syncthreads();
    if (lane == 63) sh[w] = x;
    __syncthreads();
    uint32_t base = 0, tot = 0;
    for (int i = 0; i < nw; i++) { if (i < w) base += sh[i]; tot += sh[i]; }
    *total = tot;
    return base + x - v;
}

// ------------------------------------------------------------------ alphabet
// Direct mode (live width w <= 16 bits): a 2^16-bit presence bitmap.
template <int ES>
__global__ void __launch_bounds__(RT) alpha_mark_direct(const uint8_t* __restrict__ words, uint64_t n, uint32_t k,
                                                        uint32_t* __restrict__ bitmap) {
    __shared__ uint32_t bm[2048];
    for (int j = threadIdx.x; j < 2048; j += RT) bm[j] = 0;
    __syncthreads();
    for (uint64_t i = (uint64_t)blockIdx.x * RT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * RT) {
        const uint32_t v = load_word<ES>(words, i) >> k;
        const uint32_t bit = 1u << (v & 31);
        if (!(bm[v >> 5] & bit)) atomicOr(&bm[v >> 5], bit);
    }
    __syncthreads();
    for (int j = threadIdx.x; j < 2048; j += RT)
        if (bm[j]) atomicOr(&bitmap[j], bm[j]);
}

// Ranks: rank[v] for the 2^w values (NONE if absent), sym[rank] = v << k.
__global__ void __launch_bounds__(SCAN_T) alpha_rank_direct(const uint32_t* __restrict__ bitmap, uint32_t w,
                                                            uint32_t k, uint32_t* __restrict__ rank,
                                                            uint64_t* __restrict__ sym, RepairCtl* ctl) {
    __shared__ uint32_t sh[16];
    const uint32_t t = threadIdx.x;
    const uint32_t b0 = bitmap[2 * t], b1 = bitmap[2 * t + 1];
    uint32_t total;
    uint32_t base = block_excl_scan(__popc(b0) + __popc(b1), sh, &total);
    const uint32_t nv = 1u << w;
    for (uint32_t j = 0; j < 64; j++) {
        const uint32_t v = 64 * t + j;
        if (v >= nv) break;
        const bool present = ((j < 32 ? b0 : b1) >> (j & 31)) & 1u;
        if (present) { rank[v] = base; sym[base] = (uint64_t)v << k; base++; }
        else rank[v] = NONE;
    }
    if (t == 0) ctl->a0 = total;
}

template <int ES>
__global__ void __launch_bounds__(RT) alpha_map_direct(const uint8_t* __restrict__ words, uint64_t n, uint32_t k,
                                                       const uint32_t* __restrict__ rank, uint32_t nv,
                                                       uint32_t* __restrict__ tok) {
    extern __shared__ uint32_t lrank[];
    const bool staged = nv <= 16384;
    if (staged) {
        for (uint32_t j = threadIdx.x; j < nv; j += RT) lrank[j] = rank[j];
        __syncthreads();
    }
    for (uint64_t i = (uint64_t)blockIdx.x * RT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * RT) {
        const uint32_t v = load_word<ES>(words, i) >> k;
        tok[i] = staged ? lrank[v] : rank[v];
    }
}

// Hash mode (w > 16): open-addressing set of values, ids = rank of the slot.
__device__ __forceinline__ uint64_t vslot_find(const uint64_t* vkey, uint64_t mask, uint32_t v) {
    uint64_t s = mix32(v) & mask;
    for (uint64_t p = 0; p <= mask; p++) {
        const uint64_t cur = vkey[s];
        if (cur == (uint64_t)v) return s;
        if (cur == EMPTY_KEY) return EMPTY_KEY;
        s = (s + 1) & mask;
    }
    return EMPTY_KEY;
}

template <int ES>
__global__ void __launch_bounds__(RT) alpha_insert_hash(const uint8_t* __restrict__ words, uint64_t n, uint32_t k,
                                                        uint64_t* __restrict__ vkey, uint64_t mask, RepairCtl* ctl) {
    for (uint64_t i = (uint64_t)blockIdx.x * RT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * RT) {
        const uint64_t v = load_word<ES>(words, i) >> k;
        uint64_t s = mix32((uint32_t)v) & mask;
        bool ok = false;
        for (uint64_t p = 0; p <= mask; p++) {
            uint64_t cur = ld_relaxed(&vkey[s]);
            if (cur == EMPTY_KEY) {
                cur = atomicCAS((unsigned long long*)&vkey[s], (unsigned long long)EMPTY_KEY, (unsigned long long)v);
                if (cur == EMPTY_KEY) { ok = true; break; }
            }
            if (cur == v) { ok = true; break; }
            s = (s + 1) & mask;
        }
        if (!ok) atomicOr(&ctl->err, 1u);
    }
}

// Occupied-slot count per block of OCC_BLK slots.
__global__ void __launch_bounds__(RT) occ_count(const uint64_t* __restrict__ vkey, uint64_t cap,
                                                uint32_t* __restrict__ bcount) {
    __shared__ uint32_t sh[16];
    const uint64_t base = (uint64_t)blockIdx.x * OCC_BLK;
    uint32_t c = 0;
    for (uint32_t j = threadIdx.x; j < OCC_BLK; j += RT)
        if (base + j < cap && vkey[base + j] != EMPTY_KEY) c++;
    uint32_t tot;
    block_excl_scan(c, sh, &tot);
    if (threadIdx.x == 0) bcount[blockIdx.x] = tot;
}

// In-place exclusive scan of n u32 by one workgroup; the sum goes to *total.
__global__ void __launch_bounds__(SCAN_T) scan_single(uint32_t* __restrict__ a, uint32_t n, uint32_t* total) {
    __shared__ uint32_t sh[16];
    const uint32_t per = (n + SCAN_T - 1) / SCAN_T;
    const uint32_t lo = threadIdx.x * per, hi = min(n, lo + per);
    uint32_t s = 0;
    for (uint32_t j = lo; j < hi; j++) s += a[j];
    uint32_t tot;
    uint32_t run = block_excl_scan(s, sh, &tot);
    for (uint32_t j = lo; j < hi; j++) { const uint32_t v = a[j]; a[j] = run; run += v; }
    if (threadIdx.x == 0) *total = tot;
}

__global__ void __launch_bounds__(RT) occ_rank(const uint64_t* __restrict__ vkey, uint64_t cap,
                                               const uint32_t* __restrict__ bbase, uint32_t k,
                                               uint32_t* __restrict__ vrank, uint64_t* __restrict__ sym) {
    __shared__ uint32_t sh[16];
    const uint64_t base = (uint64_t)blockIdx.x * OCC_BLK;
    // 16 consecutive slots per thread, in slot order
    const uint64_t s0 = base + (uint64_t)threadIdx.x * (OCC_BLK / RT);
    uint32_t c = 0;
    for (uint32_t j = 0; j < OCC_BLK / RT; j++)
        if (s0 + j < cap && vkey[s0 + j] != EMPTY_KEY) c++;
    uint32_t tot;
    uint32_t r = bbase[blockIdx.x] + block_excl_scan(c, sh, &tot);
    for (uint32_t j = 0; j < OCC_BLK / RT; j++) {
        const uint64_t s = s0 + j;
        if (s >= cap) break;
        const uint64_t v = vkey[s];
        if (v != EMPTY_KEY) { vrank[s] = r; sym[r] = v << k; r++; }
    }
}

template <int ES>
__global__ void __launch_bounds__(RT) alpha_map_hash(const uint8_t* __restrict__ words, uint64_t n, uint32_t k,
                                                     const uint64_t* __restrict__ vkey, uint64_t mask,
                                                     const uint32_t* __restrict__ vrank, uint32_t* __restrict__ tok) {
    for (uint64_t i = (uint64_t)blockIdx.x * RT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * RT) {
        const uint32_t v = load_word<ES>(words, i) >> k;
        const uint64_t s = vslot_find(vkey, mask, v);
        tok[i] = (s == EMPTY_KEY) ? NONE : vrank[s];
    }
}

// Apply mode: rule symbols → ids of this tensor (NONE if a base symbol is not
// in its alphabet, or is not a masked word of this width).
__global__ void map_rules_kernel(const ckr_repair_rule* __restrict__ rules, uint32_t n_rules, uint32_t k, uint32_t w,
                                 const uint32_t* __restrict__ rank, const uint64_t* __restrict__ vkey,
                                 uint64_t vmask, const uint32_t* __restrict__ vrank, RepairCtl* ctl,
                                 uint32_t* __restrict__ rmap) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n_rules) return;
    const uint32_t a0 = ctl->a0;
    auto id_of = [&](uint64_t s) -> uint32_t {
        if (s >> 63) {
            const uint64_t j = s - (1ull << 63);
            return j < n_rules ? a0 + (uint32_t)j : NONE;
        }
        const uint64_t lowmask = k ? ((1ull << k) - 1) : 0;
        if (s & lowmask) return NONE;
        const uint64_t v = s >> k;
        if (v >> w) return NONE;
        if (rank) return rank[v];
        const uint64_t slot = vslot_find(vkey, vmask, (uint32_t)v);
        return slot == EMPTY_KEY ? NONE : vrank[slot];
    };
    rmap[3 * r + 0] = id_of(rules[r].lhs);
    rmap[3 * r + 1] = id_of(rules[r].rhs);
    rmap[3 * r + 2] = a0 + r;
}

// ------------------------------------------------------------------ pair table
__device__ void tab_add(const PairTab& t, RepairCtl* ctl, uint64_t key, uint32_t c) {
    uint64_t s = mix64(key) & t.mask;
    for (uint64_t p = 0; p <= t.mask; p++) {
        uint64_t cur = ld_relaxed(&t.key[s]);
        if (cur == EMPTY_KEY) {
            cur = atomicCAS((unsigned long long*)&t.key[s], (unsigned long long)EMPTY_KEY, (unsigned long long)key);
            if (cur == EMPTY_KEY) {
                const uint32_t idx = atomicAdd(&ctl->d, 1u);
                t.touched[idx] = (uint32_t)s;
                atomicAdd(&t.cnt[s], c);
                return;
            }
        }
        if (cur == key) { atomicAdd(&t.cnt[s], c); return; }
        s = (s + 1) & t.mask;
    }
    atomicOr(&ctl->err, 2u);
}

__device__ void tab_first(const PairTab& t, RepairCtl* ctl, uint64_t key, uint32_t pos) {
    uint64_t s = mix64(key) & t.mask;
    for (uint64_t p = 0; p <= t.mask; p++) {
        const uint64_t cur = t.key[s];
        if (cur == key) { atomicMin(&t.first[s], pos); return; }
        if (cur == EMPTY_KEY) break;
        s = (s + 1) & t.mask;
    }
    atomicOr(&ctl->err, 4u);
}

// COUNT: count every adjacent pair (a recount round).  FIRST (ties only): first
// occurrence of every pair.  INC (after a round's replacement): count the pairs
// holding the round's new symbol c.
enum PairMode { COUNT = 0, FIRST_OCC = 1, INC = 2 };

template <int MODE>
__global__ void __launch_bounds__(RT) pair_pass(const uint32_t* __restrict__ buf0, const uint32_t* __restrict__ buf1,
                                                RepairCtl* ctl, PairTab tab, uint32_t chunk) {
    constexpr bool FIRST = MODE == FIRST_OCC;
    if (ctl->done) return;
    if (MODE == COUNT && !ctl->recount) return;
    if (FIRST && (ctl->ncand <= 1 || ctl->best < 2)) return;
    if (MODE == INC && ctl->recount) return;
    const uint32_t c = ctl->c;
    const uint32_t n = ctl->n_cur;
    if (n < 2) return;
    const uint32_t np = n - 1;
    const uint64_t base = (uint64_t)blockIdx.x * chunk;
    if (base >= np) return;
    const uint32_t* tok = ctl->cur ? buf1 : buf0;
    __shared__ uint64_t ck[CACHE];
    __shared__ uint32_t cv[CACHE];
    for (int j = threadIdx.x; j < CACHE; j += RT) { ck[j] = EMPTY_KEY; cv[j] = FIRST ? NONE : 0u; }
    __syncthreads();
    const uint32_t end = (uint32_t)min<uint64_t>(base + chunk, np);
    // PAIR_UNROLL pairs per thread per step, their tokens loaded before any is
    // entered, so that the loads wait for memory together
    for (uint32_t i0 = (uint32_t)base + threadIdx.x; i0 < end; i0 += PAIR_UNROLL * RT) {
        uint64_t keys[PAIR_UNROLL];
#pragma unroll
        for (int u = 0; u < PAIR_UNROLL; u++) {
            const uint32_t i = i0 + u * RT;
            keys[u] = i < end ? ((uint64_t)tok[i] << 32) | tok[i + 1] : EMPTY_KEY;
        }
#pragma unroll
        for (int u = 0; u < PAIR_UNROLL; u++) {
            const uint32_t i = i0 + u * RT;
            if (i >= end) break;
            const uint64_t key = keys[u];
            if (MODE == INC && (uint32_t)(key >> 32) != c && (uint32_t)key != c) continue;
            uint32_t s = mix64(key) & (CACHE - 1);
            bool hit = false;
            for (int p = 0; p < CACHE_PROBES; p++) {
                uint64_t cur = ck[s];
                if (cur == EMPTY_KEY) {
                    cur = atomicCAS((unsigned long long*)&ck[s], (unsigned long long)EMPTY_KEY, (unsigned long long)key);
                    if (cur == EMPTY_KEY) cur = key;
                }
                if (cur == key) {
                    if (FIRST) atomicMin(&cv[s], i); else atomicAdd(&cv[s], 1u);
                    hit = true;
                    break;
                }
                s = (s + 1) & (CACHE - 1);
            }
            if (!hit) { if (FIRST) tab_first(tab, ctl, key, i); else tab_add(tab, ctl, key, 1u); }
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j < CACHE; j += RT) {
        const uint64_t key = ck[j];
        if (key == EMPTY_KEY) continue;
        if (FIRST) tab_first(tab, ctl, key, cv[j]);
        else tab_add(tab, ctl, key, cv[j]);
    }
}

// Ties only: the first occurrences are taken afresh for the current sequence.
__global__ void __launch_bounds__(RT) first_reset(RepairCtl* ctl, PairTab tab) {
    if (ctl->done || ctl->best < 2 || ctl->ncand <= 1) return;
    const uint32_t d = ctl->d;
    for (uint32_t j = blockIdx.x * RT + threadIdx.x; j < d; j += gridDim.x * RT) tab.first[tab.touched[j]] = NONE;
}

__global__ void __launch_bounds__(RT) sel_max(RepairCtl* ctl, PairTab tab) {
    __shared__ uint32_t sh[16];
    if (ctl->done) return;
    const uint32_t d = ctl->d;
    uint32_t m = 0;
    for (uint32_t j = blockIdx.x * RT + threadIdx.x; j < d; j += gridDim.x * RT) m = max(m, tab.cnt[tab.touched[j]]);
    m = block_reduce_max(m, sh);
    if (threadIdx.x == 0 && m) atomicMax(&ctl->best, m);
}

__global__ void __launch_bounds__(RT) sel_cand(RepairCtl* ctl, PairTab tab) {
    if (ctl->done) return;
    const uint32_t d = ctl->d, best = ctl->best;
    for (uint32_t j = blockIdx.x * RT + threadIdx.x; j < d; j += gridDim.x * RT) {
        const uint32_t s = tab.touched[j];
        if (tab.cnt[s] == best) { atomicAdd(&ctl->ncand, 1u); ctl->chosen = s; }
    }
}

__device__ __forceinline__ uint64_t bucket_count_of(const uint64_t* primes, uint32_t np, uint64_t n) {
    uint32_t lo = 0, hi = np;  // first entry >= n
    while (lo < hi) { const uint32_t mid = (lo + hi) >> 1; if (primes[mid] < n) lo = mid + 1; else hi = mid; }
    return primes[lo < np ? lo : np - 1];
}

__device__ __forceinline__ uint64_t bucket_of(uint64_t key, const uint64_t* sym, uint64_t P) {
    return ref_pair_hash(sym[key >> 32], sym[key & 0xFFFFFFFFu]) % P;
}

#define CKR_TIE_GUARD() if (ctl->done || ctl->best < 2 || ctl->ncand <= 1) return

__global__ void __launch_bounds__(RT) tie_bucket(RepairCtl* ctl, PairTab tab, const uint64_t* __restrict__ sym,
                                                 const uint64_t* __restrict__ primes, uint32_t np,
                                                 uint32_t* __restrict__ bfirst) {
    CKR_TIE_GUARD();
    const uint64_t P = bucket_count_of(primes, np, ctl->n_cur);
    const uint32_t d = ctl->d;
    for (uint32_t j = blockIdx.x * RT + threadIdx.x; j < d; j += gridDim.x * RT) {
        const uint32_t s = tab.touched[j];
        atomicMin(&bfirst[bucket_of(tab.key[s], sym, P)], tab.first[s]);
    }
}

__global__ void __launch_bounds__(RT) tie_pick(RepairCtl* ctl, PairTab tab, const uint64_t* __restrict__ sym,
                                               const uint64_t* __restrict__ primes, uint32_t np,
                                               const uint32_t* __restrict__ bfirst) {
    CKR_TIE_GUARD();
    const uint64_t P = bucket_count_of(primes, np, ctl->n_cur);
    const uint32_t d = ctl->d, best = ctl->best;
    for (uint32_t j = blockIdx.x * RT + threadIdx.x; j < d; j += gridDim.x * RT) {
        const uint32_t s = tab.touched[j];
        if (tab.cnt[s] != best) continue;
        const uint64_t v = ((uint64_t)bfirst[bucket_of(tab.key[s], sym, P)] << 32) | tab.first[s];
        atomicMax((unsigned long long*)&ctl->pick, (unsigned long long)v);
    }
}

__global__ void __launch_bounds__(RT) tie_resolve(RepairCtl* ctl, PairTab tab, const uint64_t* __restrict__ sym,
                                                  const uint64_t* __restrict__ primes, uint32_t np,
                                                  uint32_t* __restrict__ bfirst) {
    CKR_TIE_GUARD();
    const uint64_t P = bucket_count_of(primes, np, ctl->n_cur);
    const uint32_t d = ctl->d, best = ctl->best, pf = (uint32_t)ctl->pick;
    for (uint32_t j = blockIdx.x * RT + threadIdx.x; j < d; j += gridDim.x * RT) {
        const uint32_t s = tab.touched[j];
        if (tab.cnt[s] == best && tab.first[s] == pf) ctl->chosen = s;
        bfirst[bucket_of(tab.key[s], sym, P)] = NONE;
    }
}

// Build mode: record the round's rule or stop.  Apply mode: load rule `round`.
__global__ void round_commit(RepairCtl* ctl, PairTab tab, uint64_t* __restrict__ sym, ckr_repair_rule* rules,
                             const uint32_t* __restrict__ rmap, int build, uint32_t dlimit) {
    if (ctl->done) return;
    const uint32_t r = ctl->round;
    if (build) {
        const uint32_t best = ctl->best;
        if (best > ctl->max_pair) ctl->max_pair = best;
        if (ctl->n_cur < 2 || best < 2) { ctl->done = 1; return; }
        const uint64_t key = tab.key[ctl->chosen];
        const uint32_t a = (uint32_t)(key >> 32), b = (uint32_t)key, c = ctl->a0 + r;
        const uint64_t rs = (1ull << 63) + r;
        rules[r].replacement = rs;
        rules[r].lhs = sym[a];
        rules[r].rhs = sym[b];
        rules[r].frequency = best;
        sym[c] = rs;
        ctl->a = a; ctl->b = b; ctl->c = c; ctl->skip = 0;
        // the round's new pairs are (x, c) and (c, x): at most 2 per occurrence
        // of c and 2 per symbol x (the a0 + r + 1 ids so far), plus (c, c)
        const uint64_t fresh = 2ull * min((uint64_t)best, (uint64_t)ctl->a0 + r + 1u) + 1u;
        ctl->recount = 0;
        ctl->recount_next = ctl->d + fresh > dlimit ? 1u : 0u;
        // every occurrence of (a, b) is replaced or loses a token to an
        // overlapping replacement: its count after the round is 0
        tab.cnt[ctl->chosen] = 0;
    } else {
        ctl->a = rmap[3 * r]; ctl->b = rmap[3 * r + 1]; ctl->c = rmap[3 * r + 2];
        ctl->skip = (ctl->a == NONE || ctl->b == NONE) ? 1u : 0u;
        sym[ctl->c] = (1ull << 63) + r;
    }
}

// ------------------------------------------------------------------ replacement
// Segment function: for entering state q (1 = the previous token started a
// replacement, so this one is consumed), the emitted count and leaving state.
struct SegFn { uint32_t c0, c1, q; };  // q: bit0 = leaving state for q=0, bit1 = for q=1

__device__ __forceinline__ SegFn fn_compose(const SegFn& f, const SegFn& g) {  // f first, then g
    SegFn h;
    const uint32_t f0 = f.q & 1, f1 = (f.q >> 1) & 1;
    h.c0 = f.c0 + (f0 ? g.c1 : g.c0);
    h.c1 = f.c1 + (f1 ? g.c1 : g.c0);
    h.q = ((g.q >> f0) & 1) | (((g.q >> f1) & 1) << 1);
    return h;
}
__device__ __forceinline__ SegFn fn_identity() { return SegFn{0, 0, 2}; }

// Thread segment [i0, i0+SEG) ∩ [0, n) of the token sequence.
struct Seg {
    uint32_t t[SEG];
    uint32_t nxt;   // token after the segment
    uint32_t len;   // tokens inside [0, n)
    bool has_nxt;
};

__device__ __forceinline__ void load_seg(const uint32_t* tok, uint32_t n, uint32_t i0, Seg& s) {
    s.len = i0 < n ? min<uint32_t>(SEG, n - i0) : 0;
    if (s.len == SEG) {
        const uint4* p = reinterpret_cast<const uint4*>(tok + i0);
#pragma unroll
        for (int q = 0; q < SEG / 4; q++) {
            const uint4 v = p[q];
            s.t[4 * q] = v.x; s.t[4 * q + 1] = v.y; s.t[4 * q + 2] = v.z; s.t[4 * q + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < SEG; j++) s.t[j] = (uint32_t)j < s.len ? tok[i0 + j] : NONE;
    }
    s.has_nxt = i0 + SEG < n;
    s.nxt = s.has_nxt ? tok[i0 + SEG] : NONE;
}

// Does position j of the segment start a replacement (given it is not consumed)?
__device__ __forceinline__ bool starts(const Seg& s, int j, uint32_t a, uint32_t b) {
    if ((uint32_t)j >= s.len) return false;
    const bool nx = (j + 1 < SEG) ? ((uint32_t)(j + 1) < s.len) : s.has_nxt;
    const uint32_t next = (j + 1 < SEG) ? s.t[(j + 1) & (SEG - 1)] : s.nxt;
    return s.t[j] == a && nx && next == b;
}

__device__ __forceinline__ SegFn seg_fn(const Seg& s, uint32_t a, uint32_t b) {
    uint32_t q0 = 0, q1 = 1, c0 = 0, c1 = 0;
#pragma unroll
    for (int j = 0; j < SEG; j++) {
        const bool valid = (uint32_t)j < s.len;
        const bool st = starts(s, j, a, b);
        c0 += (valid && !q0) ? 1 : 0;
        c1 += (valid && !q1) ? 1 : 0;
        q0 = valid ? ((q0 || !st) ? 0 : 1) : q0;
        q1 = valid ? ((q1 || !st) ? 0 : 1) : q1;
    }
    return SegFn{c0, c1, q0 | (q1 << 1)};
}

// Inclusive scan of segment functions over the block: within each wave by
// shuffles, then the waves' totals through LDS.  Leaves thread i's inclusive
// function in sh[i].
__device__ SegFn block_fn_scan(SegFn f, SegFn* sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        SegFn g;
        g.c0 = (uint32_t)__shfl_up((int)f.c0, o);
        g.c1 = (uint32_t)__shfl_up((int)f.c1, o);
        g.q = (uint32_t)__shfl_up((int)f.q, o);
        if (lane >= o) f = fn_compose(g, f);
    }
    if (lane == 63) sh[w] = f;
    __syncthreads();
    SegFn pre = fn_identity();
    for (int i = 0; i < w; i++) pre = fn_compose(pre, sh[i]);
    f = fn_compose(pre, f);
    __syncthreads();
    sh[threadIdx.x] = f;
    __syncthreads();
    return f;
}

#define CKR_REP_GUARD() if (ctl->done || ctl->skip) return

__global__ void __launch_bounds__(RT) rep_summary(const uint32_t* __restrict__ buf0, const uint32_t* __restrict__ buf1,
                                                  RepairCtl* ctl, SegFn* __restrict__ bfun) {
    CKR_REP_GUARD();
    __shared__ SegFn sh[RT];
    const uint32_t n = ctl->n_cur;
    const uint64_t base = (uint64_t)blockIdx.x * BLK;
    if (base >= n) return;
    const uint32_t* tok = ctl->cur ? buf1 : buf0;
    Seg s;
    load_seg(tok, n, (uint32_t)base + threadIdx.x * SEG, s);
    const SegFn f = block_fn_scan(seg_fn(s, ctl->a, ctl->b), sh);
    if (threadIdx.x == RT - 1) bfun[blockIdx.x] = f;
}

// One workgroup: per-block entering state and output offset.
__global__ void __launch_bounds__(SCAN_T) rep_scan(RepairCtl* ctl, const SegFn* __restrict__ bfun,
                                                   uint32_t* __restrict__ boff) {
    CKR_REP_GUARD();
    __shared__ SegFn sh[SCAN_T];
    const uint32_t n = ctl->n_cur;
    const uint32_t nb = (n + BLK - 1) / BLK;
    const uint32_t per = (nb + SCAN_T - 1) / SCAN_T;
    const uint32_t lo = threadIdx.x * per, hi = min(nb, lo + per);
    SegFn f = fn_identity();
    for (uint32_t j = lo; j < hi; j++) f = fn_compose(f, bfun[j]);
    sh[threadIdx.x] = f;
    __syncthreads();
    for (int o = 1; o < SCAN_T; o <<= 1) {
        SegFn g = f;
        if ((int)threadIdx.x >= o) g = fn_compose(sh[threadIdx.x - o], f);
        __syncthreads();
        sh[threadIdx.x] = g;
        f = g;
        __syncthreads();
    }
    // exclusive prefix of this thread = inclusive of the previous one
    SegFn pre = threadIdx.x ? sh[threadIdx.x - 1] : fn_identity();
    uint32_t q = pre.q & 1, off = pre.c0;  // the sequence starts in state 0
    for (uint32_t j = lo; j < hi; j++) {
        boff[j] = off | (q << 31);
        const SegFn& b = bfun[j];
        off += q ? b.c1 : b.c0;
        q = (b.q >> q) & 1;
    }
    if (threadIdx.x == SCAN_T - 1) ctl->n_next = f.c0;
}

// DEC (build rounds that keep their counts): every pair of the old sequence
// with a replaced token is subtracted from the table, through an LDS cache.
template <bool DEC>
__global__ void __launch_bounds__(RT) rep_apply(uint32_t* __restrict__ buf0, uint32_t* __restrict__ buf1,
                                                RepairCtl* ctl, const uint32_t* __restrict__ boff, PairTab tab) {
    CKR_REP_GUARD();
    __shared__ SegFn sh[RT];
    __shared__ uint64_t dk[DEC ? DCACHE : 1];
    __shared__ uint32_t dv[DEC ? DCACHE : 1];
    const uint32_t n = ctl->n_cur;
    const uint64_t base = (uint64_t)blockIdx.x * BLK;
    if (base >= n) return;
    const bool dec = DEC && !ctl->recount_next;
    if (dec)
        for (int j = threadIdx.x; j < DCACHE; j += RT) { dk[j] = EMPTY_KEY; dv[j] = 0; }
    const uint32_t* tok = ctl->cur ? buf1 : buf0;
    uint32_t* out = ctl->cur ? buf0 : buf1;
    const uint32_t a = ctl->a, b = ctl->b, c = ctl->c;
    // the block's output goes through LDS (index k at k + k / 32, so that the
    // threads' runs fall in different banks) and out in coalesced stores
    __shared__ uint32_t ob[BLK + BLK / 32];
    const uint32_t i0 = (uint32_t)base + threadIdx.x * SEG;
    Seg s;
    load_seg(tok, n, i0, s);
    const SegFn f = seg_fn(s, a, b);
    block_fn_scan(f, sh);
    const SegFn pre = threadIdx.x ? sh[threadIdx.x - 1] : fn_identity();
    const SegFn whole = sh[RT - 1];
    const uint32_t bo = boff[blockIdx.x];
    const uint32_t qb = bo >> 31;
    uint32_t q = (pre.q >> qb) & 1;
    uint32_t o = qb ? pre.c1 : pre.c0;  // within the block's output
    uint32_t cons = 0;                  // bit j: token i0 + j is replaced
#pragma unroll
    for (int j = 0; j < SEG; j++) {
        const bool valid = (uint32_t)j < s.len;
        const bool st = starts(s, j, a, b);
        const bool emit = valid && !q;
        if (valid && (q || st)) cons |= 1u << j;
        if (emit) ob[o + (o >> 5)] = st ? c : s.t[j];
        o += emit ? 1 : 0;
        q = emit && st ? 1 : 0;
    }
    if (dec) {
        const uint64_t ab = ((uint64_t)a << 32) | b;
        // the token after the segment is replaced if token SEG - 1 starts a
        // replacement or if it starts one itself
        if (s.has_nxt) {
            const bool has17 = (uint64_t)i0 + SEG + 1 < n;
            const bool st16 = !q && has17 && s.nxt == a && tok[i0 + SEG + 1] == b;
            if (q || st16) cons |= 1u << SEG;
        }
#pragma unroll
        for (int j = 0; j < SEG; j++) {
            const bool pair = (uint32_t)(j + 1) < s.len || (j == SEG - 1 && s.has_nxt);
            if (!pair || ((cons >> j) & 3u) == 0) continue;
            const uint64_t key = ((uint64_t)s.t[j] << 32) | (j + 1 < SEG ? s.t[(j + 1) & (SEG - 1)] : s.nxt);
            if (key == ab) continue;  // every (a, b) is destroyed: round_commit zeroed its count
            uint32_t sl = mix64(key) & (DCACHE - 1);
            bool hit = false;
            for (int p = 0; p < CACHE_PROBES; p++) {
                uint64_t cur = dk[sl];
                if (cur == EMPTY_KEY) {
                    cur = atomicCAS((unsigned long long*)&dk[sl], (unsigned long long)EMPTY_KEY, (unsigned long long)key);
                    if (cur == EMPTY_KEY) cur = key;
                }
                if (cur == key) { atomicAdd(&dv[sl], 1u); hit = true; break; }
                sl = (sl + 1) & (DCACHE - 1);
            }
            if (!hit) tab_add(tab, ctl, key, 0u - 1u);
        }
    }
    __syncthreads();
    const uint32_t total = qb ? whole.c1 : whole.c0;
    uint32_t* ob_out = out + (bo & 0x7FFFFFFFu);
    for (uint32_t k = threadIdx.x; k < total; k += RT) ob_out[k] = ob[k + (k >> 5)];
    if (dec)
        for (int j = threadIdx.x; j < DCACHE; j += RT)
            if (dk[j] != EMPTY_KEY) tab_add(tab, ctl, dk[j], 0u - dv[j]);
}

__global__ void __launch_bounds__(RT) tab_clear(RepairCtl* ctl, PairTab tab) {
    if (ctl->done || !ctl->recount_next) return;
    const uint32_t d = ctl->d;
    for (uint32_t j = blockIdx.x * RT + threadIdx.x; j < d; j += gridDim.x * RT) {
        const uint32_t s = tab.touched[j];
        tab.key[s] = EMPTY_KEY; tab.cnt[s] = 0; tab.first[s] = NONE;
    }
}

__global__ void round_end(RepairCtl* ctl) {
    if (ctl->done) return;
    if (!ctl->skip) { ctl->n_cur = ctl->n_next; ctl->cur ^= 1u; }
    ctl->round++;
    ctl->best = 0; ctl->ncand = 0; ctl->pick = 0; ctl->skip = 0;
    if (ctl->recount_next) ctl->d = 0;  // tab_clear has emptied the table
    ctl->recount = ctl->recount_next;
    ctl->recount_next = 0;
}

__global__ void __launch_bounds__(RT) seq_out_kernel(const uint32_t* __restrict__ buf0, const uint32_t* __restrict__ buf1,
                                                     const RepairCtl* ctl, const uint64_t* __restrict__ sym,
                                                     uint64_t* __restrict__ out) {
    const uint32_t n = ctl->n_cur;
    const uint32_t* tok = ctl->cur ? buf1 : buf0;
    for (uint32_t i = blockIdx.x * RT + threadIdx.x; i < n; i += gridDim.x * RT) {
        const uint32_t t = tok[i];
        out[i] = t == NONE ? EMPTY_KEY : sym[t];
    }
}

template <typename T>
__global__ void __launch_bounds__(RT) fill_kernel(T* __restrict__ p, uint64_t n, T v) {
    for (uint64_t i = (uint64_t)blockIdx.x * RT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * RT) p[i] = v;
}

__global__ void ctl_init(RepairCtl* ctl, uint32_t n) {
    RepairCtl c = {};
    c.n_cur = n;
    c.recount = 1;  // the first round counts every pair
    *ctl = c;
}

inline uint32_t grid_for(uint64_t n, uint32_t cap = 4096) {
    const uint64_t g = (n + RT * 4 - 1) / (RT * 4);
    return (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(g, cap));
}

template <typename T>
hipError_t fill(T* p, uint64_t n, T v, hipStream_t s) {
    if (n == 0) return hipSuccess;
    CKR_LAUNCH("repair_fill_kernel", s, fill_kernel<T><<<grid_for(n), RT, 0, s>>>(p, n, v));
    return hipGetLastError();
}

}  // namespace

// ------------------------------------------------------------------ host side
RepairLayout repair_layout(uint64_t n, int es, uint32_t k, uint32_t max_rules, uint64_t n_buckets) {
    RepairLayout L{};
    const uint32_t w = 8u * (uint32_t)es - k;
    L.w = w;
    L.direct = w <= 16;
    const uint64_t nv = L.direct ? (1ull << w) : 0;
    const uint64_t amax = std::min<uint64_t>(n, 1ull << std::min<uint32_t>(w, 40)) + max_rules;
    uint64_t pairs = n > 1 ? n - 1 : 1;
    if (amax < (1ull << 32) && amax * amax < pairs) pairs = amax * amax;
    uint64_t cap = 4096;
    while (cap < 2 * pairs) cap <<= 1;
    L.pair_cap = cap;
    uint64_t vcap = 0;
    if (!L.direct) { vcap = 4096; while (vcap < 2 * std::max<uint64_t>(n, 1)) vcap <<= 1; }
    L.vcap = vcap;
    L.n_buckets = std::max<uint64_t>(n_buckets, 1);
    const uint64_t nblk = (n + BLK - 1) / BLK + 1;
    const uint64_t nocc = vcap ? (vcap + OCC_BLK - 1) / OCC_BLK : 0;
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) { const uint64_t o = off; off += (bytes + 255) / 256 * 256; return o; };
    L.o_ctl = take(sizeof(RepairCtl));
    L.o_buf0 = take(4 * std::max<uint64_t>(n, 1));
    L.o_buf1 = take(4 * std::max<uint64_t>(n, 1));
    L.o_sym = take(8 * amax);
    L.o_bitmap = take(L.direct ? 2048 * 4 : 0);
    L.o_rank = take(4 * nv);
    L.o_vkey = take(8 * vcap);
    L.o_vrank = take(4 * vcap);
    L.o_occ = take(4 * (nocc + 1));
    L.o_pkey = take(8 * cap);
    L.o_pcnt = take(4 * cap);
    L.o_pfirst = take(4 * cap);
    L.o_touched = take(4 * cap);
    L.o_bfirst = take(4 * L.n_buckets);
    L.o_primes = take(8 * kRepairMaxPrimes);
    L.o_bfun = take(sizeof(SegFn) * nblk);
    L.o_boff = take(4 * nblk);
    L.o_rules = take(sizeof(ckr_repair_rule) * std::max<uint32_t>(max_rules, 1));
    L.o_rmap = take(12 * std::max<uint32_t>(max_rules, 1));
    L.bytes = off;
    return L;
}

// Alphabet and token sequence into buf0; returns the launch status.
static hipError_t build_alphabet(const uint8_t* words, uint64_t n, int es, uint32_t k, const RepairLayout& L,
                                 uint8_t* ws, hipStream_t s) {
    auto P = [&](uint64_t o) { return ws + o; };
    RepairCtl* ctl = reinterpret_cast<RepairCtl*>(P(L.o_ctl));
    uint32_t* tok = reinterpret_cast<uint32_t*>(P(L.o_buf0));
    uint64_t* sym = reinterpret_cast<uint64_t*>(P(L.o_sym));
    const uint32_t g = grid_for(n, 2048);
    if (L.direct) {
        uint32_t* bitmap = reinterpret_cast<uint32_t*>(P(L.o_bitmap));
        uint32_t* rank = reinterpret_cast<uint32_t*>(P(L.o_rank));
        hipError_t e = fill<uint32_t>(bitmap, 2048, 0u, s);
        if (e != hipSuccess) return e;
        if (es == 2) CKR_LAUNCH("repair_alpha_kernel", s, alpha_mark_direct<2><<<g, RT, 0, s>>>(words, n, k, bitmap));
        else CKR_LAUNCH("repair_alpha_kernel", s, alpha_mark_direct<4><<<g, RT, 0, s>>>(words, n, k, bitmap));
        CKR_LAUNCH("repair_alpha_kernel", s, alpha_rank_direct<<<1, SCAN_T, 0, s>>>(bitmap, L.w, k, rank, sym, ctl));
        const uint32_t nv = 1u << L.w;
        const size_t lds = nv <= 16384 ? nv * 4 : 0;
        if (es == 2) CKR_LAUNCH("repair_alpha_kernel", s, alpha_map_direct<2><<<g, RT, lds, s>>>(words, n, k, rank, nv, tok));
        else CKR_LAUNCH("repair_alpha_kernel", s, alpha_map_direct<4><<<g, RT, lds, s>>>(words, n, k, rank, nv, tok));
    } else {
        uint64_t* vkey = reinterpret_cast<uint64_t*>(P(L.o_vkey));
        uint32_t* vrank = reinterpret_cast<uint32_t*>(P(L.o_vrank));
        uint32_t* occ = reinterpret_cast<uint32_t*>(P(L.o_occ));
        hipError_t e = fill<uint64_t>(vkey, L.vcap, EMPTY_KEY, s);
        if (e != hipSuccess) return e;
        const uint32_t nocc = (uint32_t)((L.vcap + OCC_BLK - 1) / OCC_BLK);
        CKR_LAUNCH("repair_alpha_kernel", s, alpha_insert_hash<4><<<g, RT, 0, s>>>(words, n, k, vkey, L.vcap - 1, ctl));
        CKR_LAUNCH("repair_alpha_kernel", s, occ_count<<<nocc, RT, 0, s>>>(vkey, L.vcap, occ));
        CKR_LAUNCH("repair_alpha_kernel", s, scan_single<<<1, SCAN_T, 0, s>>>(occ, nocc, &ctl->a0));
        CKR_LAUNCH("repair_alpha_kernel", s, occ_rank<<<nocc, RT, 0, s>>>(vkey, L.vcap, occ, k, vrank, sym));
        CKR_LAUNCH("repair_alpha_kernel", s, alpha_map_hash<4><<<g, RT, 0, s>>>(words, n, k, vkey, L.vcap - 1, vrank, tok));
    }
    return hipGetLastError();
}

hipError_t repair_launch(const RepairArgs& A, hipStream_t s) {
    const RepairLayout& L = A.layout;
    uint8_t* ws = A.ws;
    auto P = [&](uint64_t o) { return ws + o; };
    RepairCtl* ctl = reinterpret_cast<RepairCtl*>(P(L.o_ctl));
    uint32_t* buf0 = reinterpret_cast<uint32_t*>(P(L.o_buf0));
    uint32_t* buf1 = reinterpret_cast<uint32_t*>(P(L.o_buf1));
    uint64_t* sym = reinterpret_cast<uint64_t*>(P(L.o_sym));
    PairTab tab{reinterpret_cast<uint64_t*>(P(L.o_pkey)), reinterpret_cast<uint32_t*>(P(L.o_pcnt)),
                reinterpret_cast<uint32_t*>(P(L.o_pfirst)), reinterpret_cast<uint32_t*>(P(L.o_touched)),
                L.pair_cap - 1};
    uint32_t* bfirst = reinterpret_cast<uint32_t*>(P(L.o_bfirst));
    uint64_t* primes = reinterpret_cast<uint64_t*>(P(L.o_primes));
    SegFn* bfun = reinterpret_cast<SegFn*>(P(L.o_bfun));
    uint32_t* boff = reinterpret_cast<uint32_t*>(P(L.o_boff));
    ckr_repair_rule* rules = reinterpret_cast<ckr_repair_rule*>(P(L.o_rules));
    uint32_t* rmap = reinterpret_cast<uint32_t*>(P(L.o_rmap));
    hipError_t e;

    CKR_LAUNCH("repair_init_kernel", s, ctl_init<<<1, 1, 0, s>>>(ctl, (uint32_t)A.n));
    if ((e = build_alphabet(A.words, A.n, A.es, A.k, L, ws, s)) != hipSuccess) return e;

    const uint32_t n32 = (uint32_t)A.n;
    // pair_pass: a few workgroups per CU, each over a contiguous chunk, so that
    // the pairs every chunk shares (the frequent ones) are added to the global
    // table once per chunk, not once per 8192 pairs
    int dev = 0, ncu = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    const uint64_t pblocks = (uint64_t)std::max(ncu, 1) * PAIR_BLOCKS_PER_CU;
    const uint32_t pchunk = (uint32_t)std::max<uint64_t>(PAIR_CHUNK, ((A.n + pblocks - 1) / pblocks + 255) & ~255ull);
    const uint32_t gpair = (uint32_t)std::max<uint64_t>(1, (A.n + pchunk - 1) / pchunk);
    // rounds keep their counts while the table stays at most 3/4 full (limit 0:
    // every round recounts)
    const uint32_t dlimit =
        A.recount_each_round ? 0u : (uint32_t)std::min<uint64_t>(L.pair_cap - L.pair_cap / 4, 0xFFFFFFFFull);
    const uint32_t grep = (uint32_t)std::max<uint64_t>(1, (A.n + BLK - 1) / BLK);
    const uint32_t gsel = 512;
    if (A.build) {
        if ((e = fill<uint64_t>(tab.key, L.pair_cap, EMPTY_KEY, s)) != hipSuccess) return e;
        if ((e = fill<uint32_t>(tab.cnt, L.pair_cap, 0u, s)) != hipSuccess) return e;
        if ((e = fill<uint32_t>(tab.first, L.pair_cap, NONE, s)) != hipSuccess) return e;
        if ((e = fill<uint32_t>(bfirst, L.n_buckets, NONE, s)) != hipSuccess) return e;
        e = hipMemcpyAsync(primes, A.h_primes, 8 * A.n_primes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return e;
    } else if (A.n_rules) {
        e = hipMemcpyAsync(rules, A.h_rules, sizeof(ckr_repair_rule) * A.n_rules, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return e;
        const uint32_t* rank = L.direct ? reinterpret_cast<const uint32_t*>(P(L.o_rank)) : nullptr;
        CKR_LAUNCH("repair_commit_kernel", s,
                   map_rules_kernel<<<(A.n_rules + 63) / 64, 64, 0, s>>>(
                       rules, A.n_rules, A.k, L.w, rank, reinterpret_cast<const uint64_t*>(P(L.o_vkey)),
                       L.vcap ? L.vcap - 1 : 0, reinterpret_cast<const uint32_t*>(P(L.o_vrank)), ctl, rmap));
    }
    const uint32_t rounds = A.build ? A.max_rules : A.n_rules;
    for (uint32_t r = 0; r < rounds; r++) {
        if (A.build) {
            CKR_LAUNCH("repair_pair_kernel", s, pair_pass<COUNT><<<gpair, RT, 0, s>>>(buf0, buf1, ctl, tab, pchunk));
            CKR_LAUNCH("repair_select_kernel", s, sel_max<<<gsel, RT, 0, s>>>(ctl, tab));
            CKR_LAUNCH("repair_select_kernel", s, sel_cand<<<gsel, RT, 0, s>>>(ctl, tab));
            CKR_LAUNCH("repair_tie_kernel", s, first_reset<<<gsel, RT, 0, s>>>(ctl, tab));
            CKR_LAUNCH("repair_tie_kernel", s, pair_pass<FIRST_OCC><<<gpair, RT, 0, s>>>(buf0, buf1, ctl, tab, pchunk));
            CKR_LAUNCH("repair_tie_kernel", s, tie_bucket<<<gsel, RT, 0, s>>>(ctl, tab, sym, primes, A.n_primes, bfirst));
            CKR_LAUNCH("repair_tie_kernel", s, tie_pick<<<gsel, RT, 0, s>>>(ctl, tab, sym, primes, A.n_primes, bfirst));
            CKR_LAUNCH("repair_tie_kernel", s, tie_resolve<<<gsel, RT, 0, s>>>(ctl, tab, sym, primes, A.n_primes, bfirst));
        }
        CKR_LAUNCH("repair_commit_kernel", s,
                   round_commit<<<1, 1, 0, s>>>(ctl, tab, sym, rules, rmap, A.build, dlimit));
        CKR_LAUNCH("repair_replace_kernel", s, rep_summary<<<grep, RT, 0, s>>>(buf0, buf1, ctl, bfun));
        CKR_LAUNCH("repair_replace_kernel", s, rep_scan<<<1, SCAN_T, 0, s>>>(ctl, bfun, boff));
        if (A.build) CKR_LAUNCH("repair_replace_kernel", s, rep_apply<true><<<grep, RT, 0, s>>>(buf0, buf1, ctl, boff, tab));
        else CKR_LAUNCH("repair_replace_kernel", s, rep_apply<false><<<grep, RT, 0, s>>>(buf0, buf1, ctl, boff, tab));
        if (A.build) CKR_LAUNCH("repair_select_kernel", s, tab_clear<<<gsel, RT, 0, s>>>(ctl, tab));
        CKR_LAUNCH("repair_commit_kernel", s, round_end<<<1, 1, 0, s>>>(ctl));
        if (A.build) CKR_LAUNCH("repair_pair_kernel", s, pair_pass<INC><<<gpair, RT, 0, s>>>(buf0, buf1, ctl, tab, pchunk));
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // every 8 rounds, stop launching once the device says the grammar is done
        if (A.build && (r & 7) == 7 && r + 1 < rounds) {
            uint32_t done = 0;
            if ((e = hipMemcpyAsync(&done, &ctl->done, 4, hipMemcpyDeviceToHost, s)) != hipSuccess) return e;
            if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
            if (done) break;
        }
    }
    if (A.d_seq_out) {
        CKR_LAUNCH("repair_seq_kernel", s,
                   seq_out_kernel<<<grid_for(A.n), RT, 0, s>>>(buf0, buf1, ctl, sym, A.d_seq_out));
    }
    (void)n32;
    return hipGetLastError();
}

}  // namespace ckr
