// checkers_amd/csrc/ckr_repair.hip — tensor-group prefix-mask repair (Re-Pair
// over masked words) on the GPU.
//
// Reference: src/tensor_group_prefix_mask_repair.cpp — build_masked_sequence
// (:328-353), find_best_pair (:376-405), apply_rule (:407-426),
// build_shared_grammar (:428-457), apply_existing_grammar (:459-467).
//
// Layout.  Each masked word (word with its low k mantissa bits cleared) is
// replaced by a dense id, its rank in the tensor's alphabet; rule r gets id
// A0 + r.  sym[id] keeps the reference's 64-bit symbol (the masked word, or
// 2^63 + r) for the tie-break hash.  Ids are 16 bits wide when the alphabet,
// the rules and the tombstone fit (bf16 with all 7 mantissa bits masked: at
// most 512 words), else 32.
//
// The sequence is never compacted between rounds.  It keeps its n positions;
// a replacement of the pair at live positions (p, q) writes the new id at p
// and tombstones over the rest of the merged span, so every live token heads a
// span of positions (itself and the tombstones of what it absorbed).  Ids from
// kRepairTomb16 / kRepairTomb32 up are tombstones: the first and the last
// tombstone of a span of L positions (one position for L = 2) hold
// tomb + min(L - 1, LMAX), and the all-ones value (LMAX, long spans) sends the
// reader to len[head] and back[last position], written only for such spans.
// So the next live token after p is p + 1 or p + 1 + (tok[p + 1] - tomb), the
// previous one before p is p - 1 or p - 1 - (tok[p - 1] - tomb): one or two
// reads near p, and a replacement writes 2 to 4 tokens of the tok array (no
// other array for spans under LMAX).  Positions are monotone in the compacted
// sequence, so first occurrences compare as the reference's do.
//
// Rounds run on the device with no host synchronisation inside a batch of
// eight (one replay of a captured graph).  A build round is up to seven
// launches, each returning at once when its case does not arise:
//   rp_pairs<COUNT>  (recount rounds: the first, or when the table could pass
//                    3/4 full) every adjacent pair of live tokens counted,
//                    through a per-workgroup LDS cache of 2048 pairs in front
//                    of a global open-addressing table;
//   rp_pairs<FIRST>  (rounds where several pairs hold the top count) the first
//                    occurrence of every pair;
//   rp_tie           (one workgroup) a recount round's selection, then any tie
//                    broken as std::unordered_map's iteration order would
//                    (below) and the rule committed;
//   rp_runs          ((x, x) rounds) the run parity: which x starts an
//                    occurrence depends on how many x precede it in its run,
//                    a function of the state entering a unit of positions, so
//                    units compose; each wave leaves its unit's function;
//   rp_find          every occurrence of the pair (a, b) to a per-unit list,
//                    and the pair counts' changes around it (what the
//                    replacement destroys and creates), all read from the old
//                    sequence: with ids below 4096, two LDS histograms over the
//                    neighbour ids written out as one row per workgroup, else
//                    the LDS pair cache;
//   rp_write         the lists' occurrences replaced in place, and the count
//                    rows summed in tiles and added to the table;
//   rp_close         (one workgroup) the round closed (live count, round
//                    number, the table emptied before a recount) and the next
//                    pair selected from the kept counts, committed when no tie
//                    needs rp_pairs<FIRST>.
// An apply round is rp_runs and rp_find alone: the rules are known, so each
// kernel reads its rule (the batch's base round in ctl plus the round's place
// in the batch), and rp_find replaces each occurrence as it finds it (see
// rp_find for why that is safe when no counts are kept); the live count is
// taken once at the end.
// Selection: the largest count and the number of pairs holding it; a unique
// holder is the rule.  Ties: libstdc++ keeps one singly linked list; a node
// for an empty bucket goes to the list head, a node for a used bucket goes to
// the front of that bucket's run.  With reserve(size) no rehash happens, so
// the visit order is: buckets by decreasing time of their first insertion,
// and within a bucket pairs by decreasing time of insertion (first
// occurrence).  The winner maximises (first occurrence of any pair in its
// bucket, its own first occurrence); the bucket is hash % P with P the bucket
// count of reserve(size), taken from libstdc++ by the host.
//
// Kept counts: a pair of two old live tokens that are both untouched by the
// round's replacements stays a pair, so only the pairs around an occurrence
// change.  For an occurrence (p, q) of (a, b) → c with x = prev(p) and
// r = next(q), a != b:
//   left:  x is the second token of an earlier occurrence (x holds b and
//          prev(x) holds a): (b, a) becomes (c, c); else (x, a) becomes (x, c);
//   right: r starts an occurrence (r holds a, next(r) holds b): that one's
//          left side accounts for the pair; else (b, r) becomes (c, r);
// and a == b == x (occurrences pair up the x of a run from its start):
//   left:  x at prev(p) is a replaced second, so the new pair is (c, c); any
//          other token t: (t, x) becomes (t, c);
//   right: r holds x and starts an occurrence: nothing; r holds x and does not
//          (the odd last x of its run): (c, x) is new; else (x, r) becomes (c, r).
// Every occurrence of (a, b) is replaced or loses a token to an overlapping
// replacement, so its count is set to 0 at the commit.
#include <mutex>
#include <vector>

#include "ckr_internal.h"

namespace ckr {
namespace {

constexpr uint64_t EMPTY_KEY = ~0ull;
constexpr uint32_t NONE = 0xFFFFFFFFu;
constexpr int RT = 256;          // threads per workgroup
constexpr int CACHE = 2048;      // LDS pair cache entries
constexpr int CACHE_PROBES = 8;
constexpr int SEG = 16;          // positions per thread in rp_runs / rp_find
constexpr int BLK = RT * SEG;    // positions per seq_count / seq_write block
constexpr int SCAN_T = 1024;     // threads of the single-workgroup alphabet scan
constexpr uint32_t PAIR_CHUNK = 8192;  // least positions per rp_pairs workgroup
constexpr int PAIR_UNROLL = 4;   // pairs loaded together per rp_pairs thread
constexpr uint32_t OCC_BLK = 4096;
constexpr uint32_t CHUNK = 64 * SEG;    // positions a wave takes at once
constexpr uint32_t FIND_GRID = 1024;   // rp_runs / rp_find / rp_write workgroups (4 units each)
constexpr int CLOSE_T = 1024;          // rp_close threads
constexpr uint32_t HV = 4096;          // ids up to which rp_find gathers count changes in direct LDS histograms
constexpr uint32_t MERGE_RG = 64;      // row groups of the histogram merge in rp_write

template <typename T>
__host__ __device__ __forceinline__ constexpr T tomb() { return (T)~(T)0; }
// The least tombstone id, and the span-length field's "look it up" value.
template <typename T>
__host__ __device__ __forceinline__ constexpr uint32_t tb0() { return sizeof(T) == 2 ? kRepairTomb16 : kRepairTomb32; }
template <typename T>
__host__ __device__ __forceinline__ constexpr uint32_t lmax() { return (uint32_t)tomb<T>() - tb0<T>(); }

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
__device__ __forceinline__ uint32_t ld_relaxed32(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int ES>
__device__ __forceinline__ uint32_t load_word(const uint8_t* w, uint64_t i) {
    if constexpr (ES == 2) return reinterpret_cast<const uint16_t*>(w)[i];
    else return reinterpret_cast<const uint32_t*>(w)[i];
}

// The live position after live position i (N if none), t1 being the token at
// i + 1: i + 1 itself, or past i's span, whose first tombstone (i + 1) holds
// its length (or says to read len[i]).
template <typename T>
__device__ __forceinline__ uint32_t next_from(const uint32_t* __restrict__ len, uint32_t i, uint32_t t1, uint32_t N) {
    if (i + 1 >= N) return N;
    if (t1 < tb0<T>()) return i + 1;
    const uint32_t s = t1 - tb0<T>();
    return min(s < lmax<T>() ? i + 1 + s : i + len[i], N);
}
template <typename T>
__device__ __forceinline__ uint32_t next_live(const T* __restrict__ tok, const uint32_t* __restrict__ len, uint32_t i,
                                              uint32_t N) {
    if (i + 1 >= N) return N;
    return next_from<T>(len, i, tok[i + 1], N);
}
// The live position before live position i (NONE if none), t0 being the token
// at i - 1: i - 1 itself, or the head of the span whose last tombstone it is
// (its length there, or back[i - 1]).
template <typename T>
__device__ __forceinline__ uint32_t prev_from(const uint32_t* __restrict__ back, uint32_t i, uint32_t t0) {
    if (i == 0) return NONE;
    if (t0 < tb0<T>()) return i - 1;
    const uint32_t s = t0 - tb0<T>();
    const uint32_t h = s < lmax<T>() ? (s < i ? i - 1 - s : NONE) : back[i - 1];
    return h < i ? h : NONE;  // (a head lies before its span's end)
}
template <typename T>
__device__ __forceinline__ uint32_t prev_live(const T* __restrict__ tok, const uint32_t* __restrict__ back, uint32_t i) {
    if (i == 0) return NONE;
    return prev_from<T>(back, i, tok[i - 1]);
}

struct PairTab {
    uint64_t* key;
    uint32_t* cnt;
    uint32_t* first;
    uint32_t* touched;
    uint64_t mask;  // capacity - 1 (power of two)
};

__device__ __forceinline__ uint64_t pair_key(uint32_t l, uint32_t r) { return ((uint64_t)l << 32) | r; }

// ------------------------------------------------------------------ block helpers
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
    __syncthreads();
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

template <int ES, typename T>
__global__ void __launch_bounds__(RT) alpha_map_direct(const uint8_t* __restrict__ words, uint64_t n, uint32_t k,
                                                       const uint32_t* __restrict__ rank, uint32_t nv,
                                                       T* __restrict__ tok) {
    extern __shared__ uint32_t lrank[];
    const bool staged = nv <= 16384;
    if (staged) {
        for (uint32_t j = threadIdx.x; j < nv; j += RT) lrank[j] = rank[j];
        __syncthreads();
    }
    for (uint64_t i = (uint64_t)blockIdx.x * RT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * RT) {
        const uint32_t v = load_word<ES>(words, i) >> k;
        tok[i] = (T)(staged ? lrank[v] : rank[v]);
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
                                                     const uint32_t* __restrict__ vrank, uint32_t* __restrict__ tok,
                                                     RepairCtl* ctl) {
    for (uint64_t i = (uint64_t)blockIdx.x * RT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * RT) {
        const uint32_t v = load_word<ES>(words, i) >> k;
        const uint64_t s = vslot_find(vkey, mask, v);
        if (s == EMPTY_KEY) atomicOr(&ctl->err, 1u);
        tok[i] = (s == EMPTY_KEY) ? 0u : vrank[s];
    }
}

// Apply mode: rule symbols → ids of this tensor (NONE if a base symbol is not
// in its alphabet, or is not a masked word of this width); rule r's id
// A0 + r gets its symbol 2^63 + r.
__global__ void map_rules_kernel(const ckr_repair_rule* __restrict__ rules, uint32_t n_rules, uint32_t k, uint32_t w,
                                 const uint32_t* __restrict__ rank, const uint64_t* __restrict__ vkey,
                                 uint64_t vmask, const uint32_t* __restrict__ vrank, RepairCtl* ctl,
                                 uint32_t* __restrict__ rmap, uint64_t* __restrict__ sym) {
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
    sym[a0 + r] = (1ull << 63) + r;
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

// K adds to the table at once (val 0: nothing): the home slots' keys are
// loaded together (keys only go from empty to set while the counting kernels
// run, so a plain load that finds the key is right), empty home slots are
// claimed together, and what is left (a home slot held by another key) takes
// the probing path.
template <int K>
__device__ __forceinline__ void tab_add_many(const PairTab& t, RepairCtl* ctl, const uint64_t (&key)[K],
                                             const uint32_t (&val)[K]) {
    uint64_t slot[K], cur[K];
#pragma unroll
    for (int i = 0; i < K; i++) {
        slot[i] = mix64(key[i]) & t.mask;
        cur[i] = val[i] ? t.key[slot[i]] : key[i];
    }
#pragma unroll
    for (int i = 0; i < K; i++) {
        if (!val[i] || cur[i] != EMPTY_KEY) continue;
        cur[i] = atomicCAS((unsigned long long*)&t.key[slot[i]], (unsigned long long)EMPTY_KEY,
                           (unsigned long long)key[i]);
        if (cur[i] == EMPTY_KEY) {
            t.touched[atomicAdd(&ctl->d, 1u)] = (uint32_t)slot[i];
            cur[i] = key[i];
        }
    }
#pragma unroll
    for (int i = 0; i < K; i++) {
        if (!val[i]) continue;
        if (cur[i] == key[i]) atomicAdd(&t.cnt[slot[i]], val[i]);
        else tab_add(t, ctl, key[i], val[i]);
    }
}

// LDS cache of pair updates in front of the global table: adds (FIRST: the
// least position) accumulate per key, misses go to the table directly.
template <bool FIRST>
__device__ __forceinline__ void cache_put(uint64_t* ck, uint32_t* cv, const PairTab& tab, RepairCtl* ctl,
                                          uint64_t key, uint32_t v) {
    uint32_t s = (uint32_t)mix64(key) & (CACHE - 1);
    for (int p = 0; p < CACHE_PROBES; p++) {
        uint64_t cur = ck[s];
        if (cur == EMPTY_KEY) {
            cur = atomicCAS((unsigned long long*)&ck[s], (unsigned long long)EMPTY_KEY, (unsigned long long)key);
            if (cur == EMPTY_KEY) cur = key;
        }
        if (cur == key) {
            if (FIRST) atomicMin(&cv[s], v); else atomicAdd(&cv[s], v);
            return;
        }
        s = (s + 1) & (CACHE - 1);
    }
    if (FIRST) tab_first(tab, ctl, key, v); else tab_add(tab, ctl, key, v);
}
template <bool FIRST>
__device__ void cache_init(uint64_t* ck, uint32_t* cv) {
    for (int j = threadIdx.x; j < CACHE; j += RT) { ck[j] = EMPTY_KEY; cv[j] = FIRST ? NONE : 0u; }
    __syncthreads();
}
template <bool FIRST>
__device__ void cache_flush(const uint64_t* ck, const uint32_t* cv, const PairTab& tab, RepairCtl* ctl) {
    __syncthreads();
    // A thread's CACHE / RT entries go out together: their home slots' keys are
    // loaded at once (keys only go from empty to set while the counting kernels
    // run, so a plain load that finds the key is right; one that finds anything
    // else takes the probing path), then the adds.  Each workgroup starts at its
    // own slot, so that the workgroups' updates of the same frequent pairs do not
    // all reach the table at the same moment.
    constexpr int PER = CACHE / RT;
    uint64_t key[PER], slot[PER], cur[PER];
    uint32_t val[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int j = (threadIdx.x + i * RT + blockIdx.x * 97) & (CACHE - 1);
        key[i] = ck[j];
        val[i] = cv[j];
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        slot[i] = mix64(key[i]) & tab.mask;
        cur[i] = key[i] != EMPTY_KEY ? tab.key[slot[i]] : EMPTY_KEY;
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        if (key[i] == EMPTY_KEY || (!FIRST && val[i] == 0)) continue;
        if (cur[i] == key[i]) {
            if (FIRST) atomicMin(&tab.first[slot[i]], val[i]);
            else atomicAdd(&tab.cnt[slot[i]], val[i]);
        } else if (FIRST) {
            tab_first(tab, ctl, key[i], val[i]);
        } else {
            tab_add(tab, ctl, key[i], val[i]);
        }
    }
}

// ------------------------------------------------------------------ round control (one workgroup)
__device__ __forceinline__ uint64_t bucket_count_of(const uint64_t* primes, uint32_t np, uint64_t n) {
    uint32_t lo = 0, hi = np;  // first entry >= n
    while (lo < hi) { const uint32_t mid = (lo + hi) >> 1; if (primes[mid] < n) lo = mid + 1; else hi = mid; }
    return primes[lo < np ? lo : np - 1];
}

__device__ __forceinline__ uint64_t bucket_of(uint64_t key, const uint64_t* sym, uint64_t P) {
    return ref_pair_hash(sym[key >> 32], sym[key & 0xFFFFFFFFu]) % P;
}

struct RoundArgs {
    PairTab tab;
    uint64_t* sym;
    ckr_repair_rule* rules;
    const uint32_t* rmap;
    const uint64_t* primes;
    uint32_t n_primes;
    uint32_t* bfirst;
    uint32_t rounds;   // rules to build / apply
    uint32_t dlimit;   // build: recount when the table could pass this many pairs (0: every round)
    int build;
};

// Build: record the round's rule (or stop: best count < 2).  Thread 0 only.
__device__ void commit_rule(RepairCtl* ctl, const RoundArgs& A) {
    const uint32_t r = ctl->round;
    const uint32_t best = ctl->best;
    if (r >= A.rounds) { ctl->done = 1; return; }  // the last rule is built: no round r is counted
    if (best > ctl->max_pair) ctl->max_pair = best;
    if (ctl->n_cur < 2 || best < 2) { ctl->done = 1; return; }
    const uint64_t key = A.tab.key[ctl->chosen];
    const uint32_t a = (uint32_t)(key >> 32), b = (uint32_t)key, c = ctl->a0 + r;
    const uint64_t rs = (1ull << 63) + r;
    A.rules[r].replacement = rs;
    A.rules[r].lhs = A.sym[a];
    A.rules[r].rhs = A.sym[b];
    A.rules[r].frequency = best;
    A.sym[c] = rs;
    ctl->a = a; ctl->b = b; ctl->c = c; ctl->skip = 0; ctl->tie = 0;
    ctl->run_mode = a == b ? 1u : 0u;
    // the round's new pairs are (x, c) and (c, x): at most 2 per occurrence
    // of c and 2 per symbol x (the a0 + r + 1 ids so far), plus (c, c)
    const uint64_t fresh = 2ull * min((uint64_t)best, (uint64_t)ctl->a0 + r + 1u) + 1u;
    ctl->recount = 0;
    ctl->recount_next = (uint64_t)ctl->d + fresh > A.dlimit ? 1u : 0u;
    A.tab.cnt[ctl->chosen] = 0;
}

// The pair of the round a grid kernel works on.  Build: the one committed in
// ctl (by rp_close or the tie-break).  Apply: rule ctl->round + ri of the
// mapped rules, ri being the round's place in its batch (ctl->round moves once
// per batch), so that apply rounds need no closing launch.
struct RoundSel {
    const uint32_t* rmap;  // apply: (a, b, c) per rule; null in build
    uint32_t rounds;       // apply: rule count
    uint32_t ri;           // apply: the round's index within its batch
};
struct Cur {
    uint32_t a, b, c;
    bool live, run;  // live: there is a pair to replace
};
__device__ __forceinline__ Cur cur_round(const RepairCtl* ctl, const RoundSel& rs) {
    Cur x;
    if (!rs.rmap) {
        x.live = !ctl->done && !ctl->skip;
        x.a = ctl->a; x.b = ctl->b; x.c = ctl->c;
        x.run = ctl->run_mode != 0;
        return x;
    }
    const uint32_t r = ctl->round + rs.ri;
    x.live = r < rs.rounds;
    x.a = x.b = x.c = NONE;
    if (x.live) {
        x.a = rs.rmap[3 * r]; x.b = rs.rmap[3 * r + 1]; x.c = rs.rmap[3 * r + 2];
        x.live = x.a != NONE && x.b != NONE;
    }
    x.run = x.a == x.b;
    return x;
}

// The largest count over the table's used slots, the number of slots holding
// it and one of them, in one pass: each thread reduces its slots (four loads
// in flight), then the threads' results are combined by wave shuffles and the
// waves' through LDS.  Every thread gets the result.
struct TopCount {
    uint32_t best, n, slot;
};
__device__ __forceinline__ TopCount top_combine(TopCount x, TopCount y) {
    if (y.best > x.best) return y;
    if (y.best == x.best) x.n += y.n;
    return x;
}
__device__ TopCount table_top(RepairCtl* ctl, const PairTab& t) {
    __shared__ TopCount sw[16];
    const uint32_t d = ld_relaxed32(&ctl->d), bs = blockDim.x;
    TopCount r{0, 0, 0};
    uint32_t j = threadIdx.x;
    for (; j + 3 * bs < d; j += 4 * bs) {
        uint32_t sl[4], v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) sl[i] = t.touched[j + i * bs];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = ld_relaxed32(&t.cnt[sl[i]]);
#pragma unroll
        for (int i = 0; i < 4; i++) r = top_combine(r, TopCount{v[i], 1, sl[i]});
    }
    for (; j < d; j += bs) {
        const uint32_t sl = t.touched[j];
        r = top_combine(r, TopCount{ld_relaxed32(&t.cnt[sl]), 1, sl});
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        TopCount y;
        y.best = (uint32_t)__shfl_xor((int)r.best, o);
        y.n = (uint32_t)__shfl_xor((int)r.n, o);
        y.slot = (uint32_t)__shfl_xor((int)r.slot, o);
        r = top_combine(r, y);
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sw[threadIdx.x >> 6] = r;
    __syncthreads();
    TopCount all{0, 0, 0};
    for (uint32_t w = 0; w < bs / 64; w++) all = top_combine(all, sw[w]);
    __syncthreads();
    return all;
}

// Build: the largest count and its holders over the table's used slots; a
// unique holder (or none worth a rule) commits, several set up the tie-break
// (their first occurrences are taken by rp_pairs<FIRST>).
__device__ void select_round(RepairCtl* ctl, const RoundArgs& A) {
    const TopCount top = table_top(ctl, A.tab);
    const uint32_t ncand = top.best >= 2 ? top.n : 0u;
    if (threadIdx.x == 0) {
        ctl->best = top.best;
        ctl->ncand = ncand;
        ctl->chosen = top.slot;
        if (top.best >= 2 && ncand > 1 && ctl->n_cur >= 2) ctl->tie = 1;  // first[] is NONE outside a tie
        else commit_rule(ctl, A);
    }
    __syncthreads();
}

// Build, after rp_pairs<FIRST>: the holder of the top count that std::unordered_map
// visits first, then the commit.
__device__ void break_tie(RepairCtl* ctl, const RoundArgs& A) {
    __shared__ unsigned long long s_pick;
    __shared__ uint32_t s_chosen;
    const PairTab& t = A.tab;
    const uint64_t P = bucket_count_of(A.primes, A.n_primes, ctl->n_cur);
    const uint32_t d = ctl->d, best = ctl->best;
    for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) {
        const uint32_t s = t.touched[j];
        atomicMin(&A.bfirst[bucket_of(t.key[s], A.sym, P)], ld_relaxed32(&t.first[s]));
    }
    if (threadIdx.x == 0) { s_pick = 0; s_chosen = 0; }
    __threadfence();
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) {
        const uint32_t s = t.touched[j];
        if (t.cnt[s] != best) continue;
        const uint64_t v = ((uint64_t)ld_relaxed32(&A.bfirst[bucket_of(t.key[s], A.sym, P)]) << 32) |
                           ld_relaxed32(&t.first[s]);
        atomicMax(&s_pick, (unsigned long long)v);
    }
    __syncthreads();
    const uint32_t pf = (uint32_t)s_pick;
    for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) {
        const uint32_t s = t.touched[j];
        if (t.cnt[s] == best && ld_relaxed32(&t.first[s]) == pf) s_chosen = s;
    }
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) {
        const uint32_t s = t.touched[j];
        A.bfirst[bucket_of(t.key[s], A.sym, P)] = NONE;
        t.first[s] = NONE;  // NONE again until the next tie
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        ctl->chosen = s_chosen;
        commit_rule(ctl, A);
    }
    __syncthreads();
}

// Whether the table's top count (at least 2) is held by several pairs: the
// selection's question, asked by every workgroup of rp_pairs<FIRST> in a
// recount round (all get the same answer from the same counts).
__device__ bool table_tied(RepairCtl* ctl, const PairTab& t) {
    const TopCount top = table_top(ctl, t);
    return top.best >= 2 && top.n > 1 && ctl->n_cur >= 2;
}

// ------------------------------------------------------------------ counting passes
// COUNT (rounds that recount): every adjacent pair of live tokens; FIRST
// (tied rounds): the first occurrence of every pair.  Workgroups take
// contiguous chunks of positions; the last one to finish selects (COUNT) or
// breaks the tie (FIRST).
template <typename T, bool FIRST>
__global__ void __launch_bounds__(RT) rp_pairs(const T* __restrict__ tok, const uint32_t* __restrict__ len,
                                               uint32_t N, RepairCtl* ctl, RoundArgs A, uint32_t chunk) {
    if (ctl->done) return;
    if (FIRST) {
        // a tie found by the previous round's selection, or, in a recount round,
        // one the selection after rp_pairs<COUNT> is about to find
        if (!ctl->tie && !(ctl->recount && table_tied(ctl, A.tab))) return;
    } else if (!ctl->recount) {
        return;
    }
    __shared__ uint64_t ck[CACHE];
    __shared__ uint32_t cv[CACHE];
    cache_init<FIRST>(ck, cv);
    const uint64_t base = (uint64_t)blockIdx.x * chunk;
    const uint32_t end = (uint32_t)min<uint64_t>(base + chunk, N);
    // PAIR_UNROLL positions per thread per step, their tokens loaded before any
    // pair is entered, so that the loads wait for memory together
    for (uint32_t i0 = (uint32_t)base + threadIdx.x; i0 < end; i0 += PAIR_UNROLL * RT) {
        uint32_t l[PAIR_UNROLL], r[PAIR_UNROLL];
#pragma unroll
        for (int u = 0; u < PAIR_UNROLL; u++) {
            const uint32_t i = i0 + u * RT;
            l[u] = (i < end) ? (uint32_t)tok[i] : (uint32_t)tomb<T>();
            r[u] = (i + 1 < N && i < end) ? (uint32_t)tok[i + 1] : (uint32_t)tomb<T>();
        }
#pragma unroll
        for (int u = 0; u < PAIR_UNROLL; u++) {
            const uint32_t i = i0 + u * RT;
            if (i >= end || l[u] >= tb0<T>() || i + 1 >= N) continue;
            uint32_t rr = r[u];
            if (rr >= tb0<T>()) {  // the next head, past i's span
                const uint32_t j = next_from<T>(len, i, rr, N);
                if (j >= N) continue;
                rr = tok[j];
            }
            cache_put<FIRST>(ck, cv, A.tab, ctl, pair_key(l[u], rr), FIRST ? i : 1u);
        }
    }
    cache_flush<FIRST>(ck, cv, A.tab, ctl);
}

// One workgroup after rp_pairs<FIRST>: in a recount round the selection
// (committing a unique pair), then any tie broken and its pair committed.
__global__ void __launch_bounds__(CLOSE_T) rp_tie(RepairCtl* ctl, RoundArgs A) {
    if (ctl->done) return;
    if (ctl->recount) select_round(ctl, A);
    if (ctl->done || !ctl->tie) return;
    break_tie(ctl, A);
}

// ------------------------------------------------------------------ run parity ((x, x) rounds)
// State entering a position: 1 if the previous live token started an
// occurrence (this one is its second).  A segment of positions maps the entering
// state to the leaving one: bit q of f is the leaving state for entering q
// (identity 0b10).  Tombstones leave the state as it is.
__device__ __forceinline__ uint32_t fn_compose(uint32_t f, uint32_t g) {  // f first, then g
    return ((g >> (f & 1)) & 1) | (((g >> ((f >> 1) & 1)) & 1) << 1);
}
constexpr uint32_t FN_ID = 2;

__device__ __forceinline__ uint32_t seg_fn(uint32_t live, uint32_t st) {
    uint32_t q0 = 0, q1 = 1;
#pragma unroll
    for (int j = 0; j < SEG; j++) {
        if (!((live >> j) & 1)) continue;
        const uint32_t s = (st >> j) & 1;
        q0 = q0 ? 0 : s;
        q1 = q1 ? 0 : s;
    }
    return q0 | (q1 << 1);
}

// rp_runs, rp_find and rp_write share one partition of the sequence into
// units, one per wave: unit u takes the contiguous chunks [u K, (u + 1) K) of
// CHUNK positions (a wave's 64 lanes x SEG), K = ceil(chunks / units).  A wave
// works through its unit on its own (no workgroup barrier), lane l taking
// positions [i0, i0 + SEG) of each chunk, i0 = chunk CHUNK + l SEG.
struct Unit {
    uint32_t u, c0, c1;  // unit, its chunks [c0, c1)
};
__device__ __forceinline__ Unit unit_of(uint32_t N, uint32_t K) {
    Unit x;
    x.u = blockIdx.x * (RT / 64) + (threadIdx.x >> 6);
    const uint32_t nch = (N + CHUNK - 1) / CHUNK;
    x.c0 = min(nch, x.u * K);
    x.c1 = min(nch, x.c0 + K);
    return x;
}

// The tokens around a lane's positions, token k (k < 32) = tok[i0 - 8 + k],
// with tombstones for positions outside [0, N) (the array carries 32
// tombstones past its end), packed as loaded: R words of 32 bits.  i0 is a
// multiple of SEG, so every load is 16-byte aligned.  sel(k) takes token k
// by a tree of selects over the words, so that a run-time k needs no indexed
// register access (which would go to scratch memory); a constant k folds to
// one word.
template <typename T>
struct Win {
    static constexpr int PER = 16 / sizeof(T);  // tokens per 16-byte load
    static constexpr int R = 32 * sizeof(T) / 4;
    uint32_t r[R];
    __device__ __forceinline__ void load(const T* __restrict__ tok, uint32_t N, uint32_t i0) {
        const uint4* v = reinterpret_cast<const uint4*>(tok + i0) - 8 / PER;
#pragma unroll
        for (int q = 0; q < R / 4; q++) {
            uint4 x;
            // before position 0, or a lane wholly past the end: tombstones
            if ((q < 8 / PER && i0 == 0) || i0 >= N) x = make_uint4(~0u, ~0u, ~0u, ~0u);
            else x = v[q];
            r[4 * q] = x.x; r[4 * q + 1] = x.y; r[4 * q + 2] = x.z; r[4 * q + 3] = x.w;
        }
    }
    __device__ __forceinline__ uint32_t word_tok(uint32_t w, uint32_t k) const {
        return sizeof(T) == 4 ? w : ((w >> (16 * (k & 1))) & 0xFFFFu);
    }
    __device__ __forceinline__ uint32_t sel(uint32_t k) const {
        const uint32_t idx = sizeof(T) == 4 ? k : k >> 1;
        uint32_t t[R];
#pragma unroll
        for (int i = 0; i < R; i++) t[i] = r[i];
#pragma unroll
        for (int half = R / 2, bit = 1; half >= 1; half >>= 1, bit <<= 1) {
#pragma unroll
            for (int i = 0; i < half; i++) t[i] = (idx & bit) ? t[2 * i + 1] : t[2 * i];
        }
        return word_tok(t[0], k);
    }
    static constexpr uint32_t TB0 = tb0<T>();  // tokens from here up are tombstones
};

// Wave-wide inclusive scan of segment functions (lane order); returns this
// lane's exclusive prefix, *whole the wave's function.
__device__ __forceinline__ uint32_t wave_fn_scan(uint32_t f, uint32_t* whole) {
    const int lane = threadIdx.x & 63;
    uint32_t inc = f;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t g = (uint32_t)__shfl_up((int)inc, o);
        if (lane >= o) inc = fn_compose(g, inc);
    }
    *whole = (uint32_t)__shfl((int)inc, 63);
    const uint32_t ex = (uint32_t)__shfl_up((int)inc, 1);
    return lane ? ex : FN_ID;
}

// Live positions and, for the pair (x, x), the positions that would start an
// occurrence if not consumed, among the lane's SEG positions (window w).
template <typename T>
__device__ __forceinline__ void win_runs(const Win<T>& w, const T* __restrict__ tok, const uint32_t* __restrict__ len,
                                         uint32_t N, uint32_t i0, uint32_t x, uint32_t* live, uint32_t* st) {
    uint32_t lv = 0, s = 0;
    constexpr uint32_t TB0 = Win<T>::TB0;
#pragma unroll
    for (int j = 0; j < SEG; j++) {  // unrolled: every sel() index is a constant
        const uint32_t t = w.sel(8 + j);
        if (t >= TB0) continue;
        lv |= 1u << j;
        if (t != x || i0 + j + 1 >= N) continue;
        uint32_t nx = w.sel(9 + j);
        if (nx >= TB0) {
            const uint32_t q = next_from<T>(len, i0 + j, nx, N);
            if (q >= N) continue;
            nx = tok[q];
        }
        if (nx == x) s |= 1u << j;
    }
    *live = lv;
    *st = s;
}

// (x, x) rounds: each unit's function (the composition of its chunks'), in
// rstate[u].
template <typename T>
__global__ void __launch_bounds__(RT) rp_runs(const T* __restrict__ tok, const uint32_t* __restrict__ len, uint32_t N,
                                              uint32_t K, RepairCtl* ctl, uint32_t* __restrict__ rstate,
                                              RoundSel rs) {
    const Cur cr = cur_round(ctl, rs);
    if (!cr.live || !cr.run) return;
    const uint32_t x = cr.a;
    const Unit un = unit_of(N, K);
    const uint32_t lane = threadIdx.x & 63;
    uint32_t f = FN_ID;
    Win<T> wn;  // the next chunk's window, loaded while this one is worked on
    if (un.c0 < un.c1) wn.load(tok, N, un.c0 * CHUNK + lane * SEG);
    for (uint32_t ch = un.c0; ch < un.c1; ch++) {
        const uint32_t i0 = ch * CHUNK + lane * SEG;
        const Win<T> w = wn;
        if (ch + 1 < un.c1) wn.load(tok, N, i0 + CHUNK);
        uint32_t live, st, whole;
        win_runs<T>(w, tok, len, N, i0, x, &live, &st);
        wave_fn_scan(seg_fn(live, st), &whole);
        f = fn_compose(f, whole);
    }
    if (lane == 0) rstate[un.u] = f;
}

// ------------------------------------------------------------------ find and replace
// Every occurrence (p, q) of (a, b) in the unit: (p, q, e) to the unit's part
// of the list, e the position after q's span (the next live token or N), and
// (build rounds keeping their counts) the pair count changes around the
// occurrence (see the file comment), all read from the old sequence.  The
// neighbours come from the lane's window when they lie in it and are live,
// else from the span lengths and heads.
// The occurrence (p, q) replaced by c, its merged span [p, e) (e: the next live
// position after q, or N): the first and last tombstones of the span carry its
// length, q (when it is neither) becomes a plain tombstone.
template <typename T>
__device__ __forceinline__ void merge_span(T* tok, uint32_t* len, uint32_t* back, uint32_t p, uint32_t q, uint32_t e,
                                           T c) {
    const uint32_t L = e - p, sl = min(L - 1, lmax<T>());
    const T ts = (T)(tb0<T>() + sl);
    tok[p] = c;
    tok[p + 1] = ts;
    if (q != p + 1 && q != e - 1) tok[q] = ts;
    tok[e - 1] = ts;
    if (sl == lmax<T>()) { len[p] = L; back[e - 1] = p; }
}

// Apply rounds (BUILD false) replace each occurrence in place as they find it,
// in the same pass: every read that decides an occurrence (is p a start, where
// is q, where is r) lands on the positions of its own span or on positions
// whose old and new values lead to the same decision (a start or a live token
// stays live; a written a becomes c, and neither is b or, in (x, x) rounds,
// changes a decision the run states already fixed), and windows are loaded
// before the chunk's writes.  Build rounds read farther neighbours for the
// counts and leave the writing to rp_write.
template <typename T, bool BUILD>
__global__ void __launch_bounds__(RT) rp_find(T* tok, uint32_t* len, uint32_t* back, uint32_t N, uint32_t K,
                                              RepairCtl* ctl, PairTab tab, const uint32_t* __restrict__ rstate,
                                              uint32_t* __restrict__ ucount, uint32_t* __restrict__ lp,
                                              uint32_t* __restrict__ lq, uint32_t* __restrict__ le, uint32_t nids,
                                              uint32_t* __restrict__ hist, RoundSel rs) {
    const Cur cr = cur_round(ctl, rs);
    if (!cr.live) return;
    // count changes: with ids below nids <= HV, two histograms over the ids
    // (hl[t]: occurrences whose left neighbour t loses (t, a) and gains (t, c);
    // hr[t]: right neighbour t, (b, t) to (c, t)) and three counters for the
    // pairs of the run and overlap cases (hs: (c, c), (b, a) to (c, c), (c, a));
    // else an LDS cache of pair keys
    __shared__ uint64_t lds[HV];
    __shared__ uint32_t hs[3];
    uint64_t* ck = lds;
    uint32_t* cv = reinterpret_cast<uint32_t*>(lds + CACHE);
    uint32_t* hl = reinterpret_cast<uint32_t*>(lds);
    uint32_t* hr = hl + HV;
    constexpr uint32_t TB0 = Win<T>::TB0;
    const uint32_t a = cr.a, b = cr.b, c = cr.c;
    const bool run = cr.run;
    const bool count = BUILD && !ctl->recount_next;  // a recount follows: no count to keep
    const bool direct = nids <= HV;
    if (count) {
        if (direct) {
            for (uint32_t j = threadIdx.x; j < nids; j += RT) { hl[j] = 0; hr[j] = 0; }
            if (threadIdx.x < 3) hs[threadIdx.x] = 0;
            __syncthreads();
        } else {
            cache_init<false>(ck, cv);
        }
    }
    auto upd = [&](uint32_t l, uint32_t r, uint32_t v) { cache_put<false>(ck, cv, tab, ctl, pair_key(l, r), v); };
    const uint32_t DEC = 0u - 1u;
    auto left = [&](uint32_t t) {
        if (direct) atomicAdd(&hl[t], 1u);
        else { upd(t, a, DEC); upd(t, c, 1u); }
    };
    auto right = [&](uint32_t t) {
        if (direct) atomicAdd(&hr[t], 1u);
        else { upd(b, t, DEC); upd(c, t, 1u); }
    };
    auto cc = [&]() { if (direct) atomicAdd(&hs[0], 1u); else upd(c, c, 1u); };
    auto ba = [&]() { if (direct) atomicAdd(&hs[1], 1u); else { upd(b, a, DEC); upd(c, c, 1u); } };
    auto ca = [&]() { if (direct) atomicAdd(&hs[2], 1u); else upd(c, a, 1u); };
    const Unit un = unit_of(N, K);
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t base = (uint64_t)un.u * K * (CHUNK / 2);  // the unit's slots: at most CHUNK / 2 per chunk
    uint32_t wcount = 0;                                      // slots used (uniform over the wave)
    uint32_t qw = 0;                                          // state entering the chunk
    if (run) {
        // the state entering this wave's unit: the units before it composed
        // (rp_runs left each unit's function in rstate), the sequence starting
        // in state 0.  The workgroup composes the units before its first
        // unit together, in order; each wave then adds the ones before its own.
        __shared__ uint32_t swf[RT / 64];
        const uint32_t u0 = blockIdx.x * (RT / 64);
        const uint32_t per = (u0 + RT - 1) / RT;
        const uint32_t lo = min(u0, threadIdx.x * per), hi = min(u0, lo + per);
        uint32_t f = FN_ID;
        for (uint32_t j = lo; j < hi; j++) f = fn_compose(f, rstate[j]);
        uint32_t whole;
        wave_fn_scan(f, &whole);
        if (lane == 0) swf[threadIdx.x >> 6] = whole;
        __syncthreads();
        uint32_t all = FN_ID;
        for (int i = 0; i < RT / 64; i++) all = fn_compose(all, swf[i]);
        qw = all & 1;
        for (uint32_t v = u0; v < un.u; v++) qw = (rstate[v] >> qw) & 1;
    }
    Win<T> wn;  // the next chunk's window, loaded while this one is worked on
    if (un.c0 < un.c1) wn.load(tok, N, un.c0 * CHUNK + lane * SEG);
    for (uint32_t ch = un.c0; ch < un.c1; ch++) {
        const uint32_t i0 = ch * CHUNK + lane * SEG;
        const Win<T> w = wn;
        if (ch + 1 < un.c1) wn.load(tok, N, i0 + CHUNK);
        uint32_t starts = 0;
        if (run) {
            uint32_t live, st, whole;
            win_runs<T>(w, tok, len, N, i0, a, &live, &st);
            const uint32_t pre = wave_fn_scan(seg_fn(live, st), &whole);
            uint32_t q = (pre >> qw) & 1;
#pragma unroll
            for (int j = 0; j < SEG; j++) {
                if (!((live >> j) & 1)) continue;
                const uint32_t s0 = q ? 0u : ((st >> j) & 1);
                starts |= s0 << j;
                q = s0;
            }
            qw = (whole >> qw) & 1;
        } else {
#pragma unroll
            for (int j = 0; j < SEG; j++) {  // unrolled: every sel() index is a constant
                if (w.sel(8 + j) != a || i0 + j + 1 >= N) continue;
                uint32_t nx = w.sel(9 + j);
                if (nx >= TB0) {
                    const uint32_t q = next_from<T>(len, i0 + j, nx, N);
                    if (q >= N) continue;
                    nx = tok[q];
                }
                if (nx == b) starts |= 1u << j;
            }
        }
        // slots (build): the wave's exclusive prefix of the lanes' counts
        uint64_t k = 0;
        if constexpr (BUILD) {
            const uint32_t nst = __popc(starts);
            uint32_t inc = nst;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t g = (uint32_t)__shfl_up((int)inc, o);
                if ((int)lane >= o) inc += g;
            }
            const uint32_t total = (uint32_t)__shfl((int)inc, 63);
            k = base + wcount + inc - nst;
            wcount += total;
        }
        // each lane through its own occurrences; neighbours from the window
        // (k - 8 relative to i0) when they lie in it and are live
        uint32_t m = starts;
        while (m) {
            const uint32_t j = __ffs(m) - 1;
            m &= m - 1;
            const uint32_t p = i0 + j;
            // q: the next live position after p (p + 1 < N: p starts an occurrence)
            const uint32_t q = next_from<T>(len, p, w.sel(9 + j), N);
            // r: the next live position after q (the end of the merged span)
            uint32_t r, tr = 0;
            if (q == p + 1) {
                const uint32_t w10 = w.sel(10 + j);
                r = next_from<T>(len, q, w10, N);
                if (r == p + 2) tr = w10;
                else if (r < N) tr = tok[r];
            } else {
                r = next_live<T>(tok, len, q, N);
                if (r < N) tr = tok[r];
            }
            if constexpr (!BUILD) {
                merge_span<T>(tok, len, back, p, q, r, (T)c);
                continue;
            }
            lp[k] = p; lq[k] = q; le[k] = r;
            k++;
            if (!count) continue;
            // x: the live position before p
            uint32_t x = NONE, tx = 0;
            if (p > 0) {
                const uint32_t w7 = w.sel(7 + j);
                x = prev_from<T>(back, p, w7);
                if (x == p - 1) tx = w7;
                else if (x != NONE) tx = tok[x];
            }
            // the token after r (only asked when r holds a)
            auto after_r = [&]() -> uint32_t {
                if (r == p + 2) {
                    const uint32_t w11 = w.sel(11 + j);
                    const uint32_t nr = next_from<T>(len, r, w11, N);
                    return nr == r + 1 ? w11 : nr < N ? (uint32_t)tok[nr] : NONE;
                }
                const uint32_t nr = next_live<T>(tok, len, r, N);
                return nr < N ? (uint32_t)tok[nr] : NONE;
            };
            if (run) {  // (b == a)
                if (x != NONE) {
                    if (tx == a) cc();
                    else left(tx);
                }
                if (r < N) {
                    if (tr == a) {
                        if (after_r() != a) ca();
                    } else {
                        right(tr);
                    }
                }
            } else {
                if (x != NONE) {
                    bool second = false;
                    if (tx == b) {
                        uint32_t txx = NONE;
                        if (x == p - 1) {
                            const uint32_t w6 = w.sel(6 + j);
                            const uint32_t xx = prev_from<T>(back, x, w6);
                            if (xx == x - 1) txx = w6;
                            else if (xx != NONE) txx = tok[xx];
                        } else {
                            const uint32_t xx = prev_live<T>(tok, back, x);
                            if (xx != NONE) txx = tok[xx];
                        }
                        second = txx == a;
                    }
                    if (second) ba();
                    else left(tx);
                }
                if (r < N && !(tr == a && after_r() == b)) right(tr);
            }
        }
    }
    if (BUILD && lane == 0) ucount[un.u] = wcount;
    if (!count) return;
    if (!direct) {
        cache_flush<false>(ck, cv, tab, ctl);
        return;
    }
    // the histograms as this workgroup's row (hl | hr | hs), summed over the
    // workgroups and added to the table by rp_write
    __syncthreads();
    uint32_t* row = hist + (uint64_t)blockIdx.x * (2 * nids + 3);
    for (uint32_t j = threadIdx.x; j < nids; j += RT) {
        row[j] = hl[j];
        row[nids + j] = hr[j];
    }
    if (threadIdx.x < 3) row[2 * nids + threadIdx.x] = hs[threadIdx.x];
}

// The round's occurrences replaced in place (no two share a position): each
// wave writes its unit's, whose positions lie in the unit's chunks.  Build
// rounds that keep counts with ids below HV (merge): the count-change rows that
// rp_find left (one per workgroup: hl | hr | hs) are summed in tiles of 256
// columns x a group of rows, and each tile's sums go to the table, so each
// pair takes one add per row group rather than one per workgroup.
template <typename T>
__global__ void __launch_bounds__(RT) rp_write(T* __restrict__ tok, uint32_t* __restrict__ len,
                                               uint32_t* __restrict__ back, uint32_t N, uint32_t K, RepairCtl* ctl,
                                               const uint32_t* __restrict__ ucount, const uint32_t* __restrict__ lp,
                                               const uint32_t* __restrict__ lq, const uint32_t* __restrict__ le,
                                               const uint32_t* __restrict__ hist, uint32_t nids, uint32_t nrows,
                                               PairTab tab, int merge, RoundSel rs) {
    const Cur cr = cur_round(ctl, rs);
    if (!cr.live) return;
    const T c = (T)cr.c;
    const Unit un = unit_of(N, K);
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t base = (uint64_t)un.u * K * (CHUNK / 2);
    const uint32_t m = ucount[un.u];
    for (uint32_t k = lane; k < m; k += 64) {
        const uint32_t p = lp[base + k], q = lq[base + k], e = le[base + k];
        if (p >= q || q >= e || e > N) continue;  // (never: p < q < e <= N)
        merge_span<T>(tok, len, back, p, q, e, c);
    }
    if (!merge || ctl->recount_next) return;
    const uint32_t a = cr.a, b = cr.b;
    const uint32_t rowlen = 2 * nids + 3, ncb = (rowlen + RT - 1) / RT;
    const uint32_t ngrp = min(MERGE_RG, nrows), rpt = (nrows + ngrp - 1) / ngrp;
    const uint32_t ntiles = ncb * ngrp;  // tiles of RT columns x rpt rows
    // a workgroup takes up to four tiles at a time (when there are more tiles
    // than workgroups), their table adds issued together
    for (uint32_t t0 = blockIdx.x; t0 < ntiles; t0 += 4 * gridDim.x) {
        uint64_t key[8];
        uint32_t val[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t tile = t0 + i * gridDim.x;
            const uint32_t col = (tile % ncb) * RT + threadIdx.x;
            const uint32_t r0 = (tile / ncb) * rpt, r1 = tile < ntiles ? min(nrows, r0 + rpt) : 0u;
            uint32_t sum = 0;
            if (col < rowlen) {
                uint32_t r = r0;
                for (; r + 4 <= r1; r += 4) {
                    const uint32_t* h = hist + (uint64_t)r * rowlen + col;
                    sum += h[0] + h[rowlen] + h[2 * rowlen] + h[3 * rowlen];
                }
                for (; r < r1; r++) sum += hist[(uint64_t)r * rowlen + col];
            }
            uint64_t k0 = 0, k1 = 0;
            uint32_t v0 = 0u - sum, v1 = sum;
            if (col < nids) {                       // left neighbour col: (col, a) to (col, c)
                k0 = pair_key(col, a); k1 = pair_key(col, c);
            } else if (col < 2 * nids) {            // right neighbour: (b, t) to (c, t)
                k0 = pair_key(b, col - nids); k1 = pair_key(c, col - nids);
            } else if (col == 2 * nids) {           // (c, c) made by runs
                k0 = k1 = pair_key(c, c); v0 = 0;
            } else if (col == 2 * nids + 1) {       // (b, a) to (c, c)
                k0 = pair_key(b, a); k1 = pair_key(c, c);
            } else {                                // (c, a) after an odd run
                k0 = k1 = pair_key(c, a); v0 = 0;
            }
            key[2 * i] = k0; key[2 * i + 1] = k1;
            val[2 * i] = v0; val[2 * i + 1] = v1;
        }
        tab_add_many<8>(tab, ctl, key, val);
    }
}

// Build, one workgroup: the round closed (live count, round number, the table
// emptied before a recount), then the next round's pair selected from the kept
// counts (committed when no tie needs rp_pairs<FIRST>).
__global__ void __launch_bounds__(CLOSE_T) rp_close(uint32_t nb, RepairCtl* ctl, const uint32_t* __restrict__ bcount,
                                                    RoundArgs A) {
    if (ctl->done) return;
    __shared__ uint32_t sh[16];
    __shared__ uint32_t s_recount;
    uint32_t occ = 0;
    if (!ctl->skip) {
        uint32_t j = threadIdx.x;
        for (; j + 3 * CLOSE_T < nb; j += 4 * CLOSE_T)
            occ += bcount[j] + bcount[j + CLOSE_T] + bcount[j + 2 * CLOSE_T] + bcount[j + 3 * CLOSE_T];
        for (; j < nb; j += CLOSE_T) occ += bcount[j];
    }
    uint32_t total;
    block_excl_scan(occ, sh, &total);
    if (threadIdx.x == 0) {
        ctl->n_cur -= total;
        ctl->round++;
        ctl->best = 0; ctl->ncand = 0; ctl->pick = 0; ctl->skip = 0; ctl->tie = 0; ctl->run_mode = 0;
        ctl->recount = ctl->recount_next;
        ctl->recount_next = 0;
        s_recount = ctl->recount;
    }
    __syncthreads();
    if (s_recount) {  // rp_pairs fills the table again
        const uint32_t d = ctl->d;
        for (uint32_t j = threadIdx.x; j < d; j += blockDim.x) {
            const uint32_t s = A.tab.touched[j];
            A.tab.key[s] = EMPTY_KEY; A.tab.cnt[s] = 0; A.tab.first[s] = NONE;
        }
        __syncthreads();
        if (threadIdx.x == 0) ctl->d = 0;
    } else {
        select_round(ctl, A);
    }
}

// Apply, after a batch of rounds: the batch's rounds are done.
__global__ void rp_batch_end(RepairCtl* ctl, uint32_t rounds) { ctl->round += rounds; }

// ------------------------------------------------------------------ output
// The live tokens as reference symbols, in order: per block of BLK positions
// the live count, one scan, then the writes.
template <typename T>
__global__ void __launch_bounds__(RT) seq_count(const T* __restrict__ tok, uint32_t N, uint32_t* __restrict__ bcount) {
    __shared__ uint32_t sh[16];
    const uint32_t i0 = blockIdx.x * BLK + threadIdx.x * SEG;
    uint32_t c = 0;
    for (int j = 0; j < SEG; j++) c += (i0 + j < N && tok[i0 + j] < tb0<T>()) ? 1u : 0u;
    uint32_t tot;
    block_excl_scan(c, sh, &tot);
    if (threadIdx.x == 0) bcount[blockIdx.x] = tot;
}

template <typename T>
__global__ void __launch_bounds__(RT) seq_write(const T* __restrict__ tok, uint32_t N,
                                                const uint32_t* __restrict__ bbase, const uint64_t* __restrict__ sym,
                                                uint64_t* __restrict__ out) {
    __shared__ uint32_t sh[16];
    const uint32_t i0 = blockIdx.x * BLK + threadIdx.x * SEG;
    uint32_t c = 0;
    for (int j = 0; j < SEG; j++) c += (i0 + j < N && tok[i0 + j] < tb0<T>()) ? 1u : 0u;
    uint32_t tot;
    uint32_t o = bbase[blockIdx.x] + block_excl_scan(c, sh, &tot);
    for (int j = 0; j < SEG; j++) {
        if (i0 + j >= N) break;
        const T t = tok[i0 + j];
        if (t < tb0<T>()) out[o++] = sym[t];
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
namespace {
// The units of rp_runs / rp_find / rp_write: at most FIND_GRID workgroups of
// four waves, each unit K chunks.
struct FindGeom {
    uint32_t nch, G, U, K;
};
FindGeom find_geom(uint64_t n) {
    FindGeom g;
    g.nch = (uint32_t)std::max<uint64_t>(1, (n + CHUNK - 1) / CHUNK);
    g.G = std::min<uint32_t>(FIND_GRID, (g.nch + 3) / 4);
    g.U = 4 * g.G;
    g.K = (g.nch + g.U - 1) / g.U;
    return g;
}
}  // namespace

RepairLayout repair_layout(uint64_t n, int es, uint32_t k, uint32_t max_rules, uint64_t n_buckets) {
    RepairLayout L{};
    const uint32_t w = 8u * (uint32_t)es - k;
    L.w = w;
    L.direct = w <= 16;
    // ids 0 .. alphabet + rules - 1, and the tombstone (all ones)
    L.tok16 = L.direct && (1ull << w) + max_rules <= kRepairTomb16;
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
    const uint64_t nn = std::max<uint64_t>(n, 1);
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) { const uint64_t o = off; off += (bytes + 255) / 256 * 256; return o; };
    L.o_ctl = take(sizeof(RepairCtl));
    L.o_tok = take((L.tok16 ? 2 : 4) * nn + 128);  // 32 tombstones past the end
    L.o_len = take(4 * nn);
    L.o_back = take(4 * nn);
    const FindGeom fg = find_geom(n);
    L.list_entries = (uint64_t)fg.U * fg.K * (CHUNK / 2);
    L.o_list = take(12 * L.list_entries);  // p, q and e of each occurrence
    L.o_bcount = take(4 * fg.U);
    L.o_sym = take(8 * amax);
    L.o_bitmap = take(L.direct ? 2048 * 4 : 0);
    L.o_rank = take(4 * nv);
    L.o_vkey = take(8 * vcap);
    L.o_vrank = take(4 * vcap);
    L.o_occ = take(4 * (std::max<uint64_t>(nocc, nblk) + 1));
    L.o_pkey = take(8 * cap);
    L.o_pcnt = take(4 * cap);
    L.o_pfirst = take(4 * cap);
    L.o_touched = take(4 * cap);
    L.o_bfirst = take(4 * L.n_buckets);
    L.o_primes = take(8 * kRepairMaxPrimes);
    L.o_bfun = take(4 * (uint64_t)fg.U);
    // ids: the alphabet (at most n words, at most 2^w), then one per rule
    L.nids = (uint32_t)std::min<uint64_t>(std::min<uint64_t>(n, 1ull << std::min<uint32_t>(w, 40)) + max_rules,
                                          0xFFFFFFFFull);
    L.hist_rows = L.nids <= HV ? fg.G : 0;
    L.hist_len = L.nids <= HV ? 2 * L.nids + 3 : 0;
    L.o_hist = take(4ull * L.hist_rows * L.hist_len);
    L.o_rules = take(sizeof(ckr_repair_rule) * std::max<uint32_t>(max_rules, 1));
    L.o_rmap = take(12 * std::max<uint32_t>(max_rules, 1));
    L.bytes = off;
    return L;
}

namespace {

// Alphabet and token sequence; returns the launch status.
template <typename T>
hipError_t build_alphabet(const uint8_t* words, uint64_t n, int es, uint32_t k, const RepairLayout& L, uint8_t* ws,
                          hipStream_t s) {
    auto P = [&](uint64_t o) { return ws + o; };
    RepairCtl* ctl = reinterpret_cast<RepairCtl*>(P(L.o_ctl));
    T* tok = reinterpret_cast<T*>(P(L.o_tok));
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
        if (es == 2) CKR_LAUNCH("repair_alpha_kernel", s, (alpha_map_direct<2, T><<<g, RT, lds, s>>>(words, n, k, rank, nv, tok)));
        else CKR_LAUNCH("repair_alpha_kernel", s, (alpha_map_direct<4, T><<<g, RT, lds, s>>>(words, n, k, rank, nv, tok)));
    } else {
        if constexpr (sizeof(T) == 4) {
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
            CKR_LAUNCH("repair_alpha_kernel", s,
                       alpha_map_hash<4><<<g, RT, 0, s>>>(words, n, k, vkey, L.vcap - 1, vrank, tok, ctl));
        } else {
            return hipErrorInvalidValue;  // hash mode always takes 32-bit ids
        }
    }
    return hipGetLastError();
}

constexpr uint32_t kRoundBatch = 8;

// The captured graphs of a batch of rounds (kRoundBatch, or the last batch's
// remainder), keyed by what their kernels' arguments derive from (the
// workspace and its layout's inputs) and the batch length.  A graph is
// captured on a library stream, instantiated once and kept; at most
// kMaxRoundGraphs are kept (the oldest goes).
struct RoundGraphKey {
    const void* ws;
    uint64_t n;
    int es, build, device, tok16;
    uint32_t k, rounds, dlimit, batch;
    bool operator==(const RoundGraphKey& o) const {
        return ws == o.ws && n == o.n && es == o.es && build == o.build && device == o.device && tok16 == o.tok16 &&
               k == o.k && rounds == o.rounds && dlimit == o.dlimit && batch == o.batch;
    }
};
struct RoundGraph {
    RoundGraphKey key;
    hipGraph_t g;
    hipGraphExec_t x;
};
constexpr size_t kMaxRoundGraphs = 64;
std::mutex g_rg_mu;
std::vector<RoundGraph> g_rgs;

// A library stream per device, made on first use (graph capture).
hipStream_t side_stream(int dev, std::vector<hipStream_t>& v) {
    if ((int)v.size() <= dev) v.resize(dev + 1, nullptr);
    if (!v[dev] && hipStreamCreateWithFlags(&v[dev], hipStreamNonBlocking) != hipSuccess) {
        (void)hipGetLastError();
        v[dev] = nullptr;
    }
    return v[dev];
}

template <typename BatchFn>
hipGraphExec_t round_graph(const RepairArgs& A, const RepairLayout& L, uint32_t len, BatchFn& batch) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) { (void)hipGetLastError(); return nullptr; }
    const RoundGraphKey key{A.ws, A.n, A.es, A.build, dev, L.tok16 ? 1 : 0, A.k, A.build ? A.max_rules : A.n_rules,
                            A.recount_each_round ? 1u : 0u, len};
    std::lock_guard<std::mutex> lk(g_rg_mu);
    for (const RoundGraph& r : g_rgs)
        if (r.key == key) return r.x;
    static std::vector<hipStream_t> cap;  // one capture stream per device
    hipStream_t cs = side_stream(dev, cap);
    if (!cs) return nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t x = nullptr;
    if (hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal) != hipSuccess) { (void)hipGetLastError(); return nullptr; }
    const hipError_t e = batch(cs, len);
    const hipError_t e2 = hipStreamEndCapture(cs, &g);
    if (e != hipSuccess || e2 != hipSuccess || !g || hipGraphInstantiate(&x, g, nullptr, nullptr, 0) != hipSuccess) {
        (void)hipGetLastError();
        if (g) (void)hipGraphDestroy(g);
        return nullptr;  // the rounds are then launched one by one
    }
    if (g_rgs.size() >= kMaxRoundGraphs) {
        (void)hipDeviceSynchronize();  // the oldest graph may still run somewhere
        (void)hipGraphExecDestroy(g_rgs.front().x);
        (void)hipGraphDestroy(g_rgs.front().g);
        g_rgs.erase(g_rgs.begin());
    }
    g_rgs.push_back({key, g, x});
    return x;
}

template <typename T>
hipError_t run_rounds(const RepairArgs& A, hipStream_t s) {
    const RepairLayout& L = A.layout;
    uint8_t* ws = A.ws;
    auto P = [&](uint64_t o) { return ws + o; };
    RepairCtl* ctl = reinterpret_cast<RepairCtl*>(P(L.o_ctl));
    T* tok = reinterpret_cast<T*>(P(L.o_tok));
    uint32_t* len = reinterpret_cast<uint32_t*>(P(L.o_len));
    uint32_t* back = reinterpret_cast<uint32_t*>(P(L.o_back));
    uint64_t* sym = reinterpret_cast<uint64_t*>(P(L.o_sym));
    uint32_t* bfun = reinterpret_cast<uint32_t*>(P(L.o_bfun));
    RoundArgs R{};
    R.tab = PairTab{reinterpret_cast<uint64_t*>(P(L.o_pkey)), reinterpret_cast<uint32_t*>(P(L.o_pcnt)),
                    reinterpret_cast<uint32_t*>(P(L.o_pfirst)), reinterpret_cast<uint32_t*>(P(L.o_touched)),
                    L.pair_cap - 1};
    R.sym = sym;
    R.rules = reinterpret_cast<ckr_repair_rule*>(P(L.o_rules));
    R.rmap = reinterpret_cast<const uint32_t*>(P(L.o_rmap));
    R.primes = reinterpret_cast<const uint64_t*>(P(L.o_primes));
    R.n_primes = A.n_primes;
    R.bfirst = reinterpret_cast<uint32_t*>(P(L.o_bfirst));
    R.build = A.build;
    R.rounds = A.build ? A.max_rules : A.n_rules;
    // rounds keep their counts while the table stays at most 3/4 full (limit 0:
    // every round recounts)
    R.dlimit = A.recount_each_round ? 0u : (uint32_t)std::min<uint64_t>(L.pair_cap - L.pair_cap / 4, 0xFFFFFFFFull);
    hipError_t e;

    CKR_LAUNCH("repair_init_kernel", s, ctl_init<<<1, 1, 0, s>>>(ctl, (uint32_t)A.n));
    if ((e = build_alphabet<T>(A.words, A.n, A.es, A.k, L, ws, s)) != hipSuccess) return e;
    // 32 tombstones past the end: the windows of the last positions read them
    if ((e = fill<T>(tok + A.n, 32, tomb<T>(), s)) != hipSuccess) return e;

    const uint32_t N = (uint32_t)A.n;
    int dev = 0, ncu = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    // counting passes: a few workgroups per CU, each over a contiguous chunk, so
    // that the pairs every chunk shares (the frequent ones) reach the global
    // table once per chunk
    const uint64_t pblocks = (uint64_t)std::max(ncu, 1);  // (runs only in recount and tie rounds; exits cheaply)
    const uint32_t pchunk = (uint32_t)std::max<uint64_t>(PAIR_CHUNK, ((A.n + pblocks - 1) / pblocks + 255) & ~255ull);
    const uint32_t gpair = (uint32_t)std::max<uint64_t>(1, (A.n + pchunk - 1) / pchunk);
    const uint32_t nblk = (uint32_t)((A.n + BLK - 1) / BLK);
    const FindGeom fg = find_geom(A.n);
    const uint32_t nids = L.nids;
    uint32_t* hist = reinterpret_cast<uint32_t*>(P(L.o_hist));
    const int merge = A.build && nids <= HV && L.hist_rows >= fg.G ? 1 : 0;
    uint32_t* bcount = reinterpret_cast<uint32_t*>(P(L.o_bcount));
    uint32_t* lp = reinterpret_cast<uint32_t*>(P(L.o_list));
    uint32_t* lq = lp + L.list_entries;
    uint32_t* le = lq + L.list_entries;
    if (A.build) {
        if ((e = fill<uint64_t>(R.tab.key, L.pair_cap, EMPTY_KEY, s)) != hipSuccess) return e;
        if ((e = fill<uint32_t>(R.tab.cnt, L.pair_cap, 0u, s)) != hipSuccess) return e;
        if ((e = fill<uint32_t>(R.tab.first, L.pair_cap, NONE, s)) != hipSuccess) return e;
        if ((e = fill<uint32_t>(R.bfirst, L.n_buckets, NONE, s)) != hipSuccess) return e;
        e = hipMemcpyAsync(const_cast<uint64_t*>(R.primes), A.h_primes, 8 * A.n_primes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return e;
    } else {
        e = hipMemcpyAsync(R.rules, A.h_rules, sizeof(ckr_repair_rule) * A.n_rules, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return e;
        const uint32_t* rank = L.direct ? reinterpret_cast<const uint32_t*>(P(L.o_rank)) : nullptr;
        CKR_LAUNCH("repair_commit_kernel", s,
                   map_rules_kernel<<<(A.n_rules + 63) / 64, 64, 0, s>>>(
                       R.rules, A.n_rules, A.k, L.w, rank, reinterpret_cast<const uint64_t*>(P(L.o_vkey)),
                       L.vcap ? L.vcap - 1 : 0, reinterpret_cast<const uint32_t*>(P(L.o_vrank)), ctl,
                       const_cast<uint32_t*>(R.rmap), sym));
    }
    // One round.  Build: every kernel reads what to do from ctl, so the rounds
    // are identical launches.  Apply: the grid kernels take the round's place
    // in its batch and read the rule themselves, rp_find writes in place; no
    // write or closing launch.
    auto round = [&](hipStream_t x, uint32_t ri) -> hipError_t {
        const RoundSel rs{A.build ? nullptr : R.rmap, R.rounds, ri};
        if (A.build) {
            CKR_LAUNCH("repair_count_kernel", x, (rp_pairs<T, false><<<gpair, RT, 0, x>>>(tok, len, N, ctl, R, pchunk)));
            CKR_LAUNCH("repair_first_kernel", x, (rp_pairs<T, true><<<gpair, RT, 0, x>>>(tok, len, N, ctl, R, pchunk)));
            CKR_LAUNCH("repair_select_kernel", x, rp_tie<<<1, CLOSE_T, 0, x>>>(ctl, R));
        }
        CKR_LAUNCH("repair_runs_kernel", x, rp_runs<T><<<fg.G, RT, 0, x>>>(tok, len, N, fg.K, ctl, bfun, rs));
        if (A.build)
            CKR_LAUNCH("repair_find_kernel", x,
                       (rp_find<T, true><<<fg.G, RT, 0, x>>>(tok, len, back, N, fg.K, ctl, R.tab, bfun, bcount, lp, lq,
                                                              le, nids, hist, rs)));
        else
            CKR_LAUNCH("repair_find_kernel", x,
                       (rp_find<T, false><<<fg.G, RT, 0, x>>>(tok, len, back, N, fg.K, ctl, R.tab, bfun, bcount, lp,
                                                               lq, le, nids, hist, rs)));
        if (A.build) {
            CKR_LAUNCH("repair_write_kernel", x,
                       rp_write<T><<<fg.G, RT, 0, x>>>(tok, len, back, N, fg.K, ctl, bcount, lp, lq, le, hist, nids,
                                                       fg.G, R.tab, merge, rs));
            CKR_LAUNCH("repair_close_kernel", x, rp_close<<<1, CLOSE_T, 0, x>>>(fg.U, ctl, bcount, R));
        }
        return hipGetLastError();
    };
    auto batch = [&](hipStream_t x, uint32_t n_rounds) -> hipError_t {
        for (uint32_t i = 0; i < n_rounds; i++) {
            const hipError_t er = round(x, i);
            if (er != hipSuccess) return er;
        }
        if (!A.build) CKR_LAUNCH("repair_close_kernel", x, rp_batch_end<<<1, 1, 0, x>>>(ctl, n_rounds));
        return hipGetLastError();
    };
    // Rounds go in batches of kRoundBatch (the last one shorter), each batch
    // one launch of a graph captured once per workspace, shape and batch
    // length and kept (a round is up to 7 launches, whose host cost would
    // otherwise exceed a small tensor's GPU work).  A build reads the device's
    // done flag after each batch but the last and stops there once it is set
    // (rounds past the last rule find the grammar done and return at once).
    // While ckr_profile_begin is in effect the kernels are launched one by one.
    for (uint32_t r = 0; r < R.rounds; r += kRoundBatch) {
        const uint32_t n_rounds = std::min(kRoundBatch, R.rounds - r);
        hipGraphExec_t gx = ckr::profiling() ? nullptr : round_graph(A, L, n_rounds, batch);
        if ((e = gx ? hipGraphLaunch(gx, s) : batch(s, n_rounds)) != hipSuccess) return e;
        if (!A.build || r + kRoundBatch >= R.rounds) continue;
        uint32_t done = 0;
        if ((e = hipMemcpyAsync(&done, &ctl->done, 4, hipMemcpyDeviceToHost, s)) != hipSuccess) return e;
        if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
        if (done) break;
    }
    // the live tokens counted per block and scanned: the output's offsets, and
    // (apply, whose rounds keep no running count) the compressed length
    if (A.d_seq_out || !A.build) {
        uint32_t* occ = reinterpret_cast<uint32_t*>(P(L.o_occ));
        CKR_LAUNCH("repair_seq_kernel", s, seq_count<T><<<nblk, RT, 0, s>>>(tok, N, occ));
        CKR_LAUNCH("repair_seq_kernel", s, scan_single<<<1, SCAN_T, 0, s>>>(occ, nblk, A.build ? occ + nblk : &ctl->n_cur));
        if (A.d_seq_out)
            CKR_LAUNCH("repair_seq_kernel", s, seq_write<T><<<nblk, RT, 0, s>>>(tok, N, occ, sym, A.d_seq_out));
    }
    return hipGetLastError();
}

}  // namespace

hipError_t repair_launch(const RepairArgs& A, hipStream_t s) {
    return A.layout.tok16 ? run_rounds<uint16_t>(A, s) : run_rounds<uint32_t>(A, s);
}

}  // namespace ckr
