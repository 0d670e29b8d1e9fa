// checkers_amd/csrc/ckr_table.h — the normalisation of a 256-bin histogram into
// 12-bit slot counts, ANSCompressor::normalize_histogram
// (src/ANSCompressor.cpp:416-503), stated so that each symbol's count follows
// from comparisons with the others: one symbol per thread on the device, or a
// loop on the host, give the same counts.
//
// The reference gives every included symbol max(1, floor(max(h,1) M / total))
// slots, sorts the symbols by the fractional part of max(h,1) M / total
// (std::sort, descending, so equal parts end up in an order only libstdc++'s
// introsort fixes), and then corrects the sum: +1 to the first M - sum symbols
// of that order, or -1 to the last sum - M of them that hold more than one slot.
// Which symbols the correction reaches depends on the order of equal parts only
// when the correction's boundary falls inside a group of equal parts; then the
// counts here are marked ambiguous and the caller takes libstdc++'s own sort
// (ckr_build_table).  Otherwise the selected set is fixed by the values alone
// and the counts equal the reference's.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace ckr {

constexpr uint32_t kTabM = 4096;       // 2^12 slots
constexpr int kNormAmbiguous = 2;      // norm_fix: the order of equal parts decides

// Step 1 for a symbol of count h: its proportional slots (at least 1 when it
// is included: present, or every symbol with ensure_full) and the fractional
// part that orders the correction; inc false: no slot, not in the order.
struct NormStart {
    uint32_t norm;
    double frac;
    bool inc;
};
__host__ __device__ inline NormStart norm_start(uint32_t h, uint64_t total, bool ensure_full) {
    NormStart r{0u, 0.0, false};
    if (!ensure_full && h == 0) return r;
    const uint32_t hm = h > 1u ? h : 1u;
    const uint32_t slots = total ? (uint32_t)((uint64_t)hm * kTabM / total) : 0u;
    r.norm = slots ? slots : 1u;
    const double exact = total ? (double)hm * kTabM / (double)total : 1.0;
    r.frac = exact - (double)(int)exact;
    r.inc = true;
    return r;
}

// The sort keys of step 2: up, the fractional part of an included symbol (-1
// otherwise, below every part); down, that of an included symbol holding more
// than one slot (2 otherwise, above every part).
__host__ __device__ inline double norm_key_up(const NormStart& r) { return r.inc ? r.frac : -1.0; }
__host__ __device__ inline double norm_key_down(const NormStart& r) { return r.inc && r.norm > 1u ? r.frac : 2.0; }

// Step 2 for symbol s (step-1 count norm_s, fractional part fs, included inc_s),
// given every symbol's keys and the step-1 sum: +1, -1, 0, or kNormAmbiguous.
// The sorted order puts the symbols of larger fractional part first; s's
// position lies in [gt, gt + eq), gt counting the larger parts and eq the equal
// ones (s included).
__host__ __device__ inline int norm_fix(uint32_t norm_s, double fs, bool inc_s, const double* up, const double* down,
                                        uint32_t assigned) {
    if (!inc_s) return 0;
    if (assigned < kTabM) {  // the first rem positions get +1
        const uint32_t rem = kTabM - assigned;
        uint32_t gt = 0, eq = 0;
#pragma unroll 16
        for (uint32_t t = 0; t < 256; t++) {
            gt += up[t] > fs ? 1u : 0u;
            eq += up[t] == fs ? 1u : 0u;
        }
        if (gt + eq <= rem) return 1;
        if (gt >= rem) return 0;
        return kNormAmbiguous;
    }
    if (assigned > kTabM) {  // from the end, the last rem symbols holding more than one slot get -1
        if (norm_s <= 1u) return 0;
        const uint32_t rem = assigned - kTabM;
        uint32_t lt = 0, eq = 0;  // such symbols after s, and those equal to it
#pragma unroll 16
        for (uint32_t t = 0; t < 256; t++) {
            lt += down[t] < fs ? 1u : 0u;
            eq += down[t] == fs ? 1u : 0u;
        }
        if (lt + eq <= rem) return -1;
        if (lt >= rem) return 0;
        return kNormAmbiguous;
    }
    return 0;
}

}  // namespace ckr
