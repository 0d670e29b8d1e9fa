// checkers_amd/csrc/ckr_container.hip — the unit records of the chunked states
// file (.ansc v4): what is stored per unit instead of its 256 lane headers,
// and which of its bytes are stored.
//
// The reference has no chunked file (its .ansc v2 keeps one 4 KiB header
// block per tensor, src/ANSCompressor.cpp:721-816); this layout is this
// library's own.  A unit's lanes are of two kinds:
//   zero-plane lanes (lane t with t % es < spe): every symbol is a masked zero,
//     so the lane's stream, final state and byte count follow from the table
//     and the lane's symbol count K alone; neither header nor bytes are stored;
//   live lanes: final state and byte count are stored, bit-packed.
// Unit record, by its first byte (the kind):
//   1 raw:    the unit's bytes are stored as they are (the passthrough rule).
//   0 packed: for each live byte plane g (residues spe..es-1): u32 base = the
//             least byte count of its lanes, u8 w = bit width of (count - base);
//             then a little-endian bit stream: the live lanes' final states, 31
//             bits each, in lane order, then their (count - base), w bits each,
//             in lane order; padded to a byte.  Stored bytes: the live lanes'
//             streams in lane order.
//   2 full:   the 256 lanes' (u32 state, u32 count), and every lane's bytes:
//             used when a zero-plane lane is not the stream its K implies or a
//             live state does not fit 31 bits.
// Unit offsets and in-unit lane offsets are not stored: they are prefix sums.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "ckr_container.h"
#include "ckr_internal.h"

namespace ckr {

namespace {

constexpr int kThreads = 64;  // one wave per unit; thread j owns lanes 4j..4j+3

struct UnitView {
    uint32_t kind;                  // 0 packed, 1 raw, 2 full
    uint32_t base[4], w[4];         // per live plane (packed)
    uint32_t live_bytes, all_bytes;
};

__device__ inline uint32_t wave_min(uint32_t v) {
    for (int d = 32; d > 0; d >>= 1) v = min(v, (uint32_t)__shfl_xor(v, d, 64));
    return v;
}
__device__ inline uint32_t wave_max(uint32_t v) {
    for (int d = 32; d > 0; d >>= 1) v = max(v, (uint32_t)__shfl_xor(v, d, 64));
    return v;
}
__device__ inline uint32_t wave_sum(uint32_t v) {
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

// The unit's kind and per-plane bases and widths, from this thread's 4 lane
// headers h[0..3] (lanes 4j..4j+3); every thread of the wave gets the result.
__device__ UnitView analyse_unit(const uint4 h[4], uint32_t len, int es, int spe, const ZeroLaneArg& z) {
    const int j = threadIdx.x;
    UnitView v{};
    bool raw = true, odd = false;
    uint32_t mn[4] = {~0u, ~0u, ~0u, ~0u}, mx[4] = {0, 0, 0, 0};
    uint32_t live = 0, all = 0;
    for (int i = 0; i < 4; i++) {
        const uint32_t t = 4 * j + i;
        const uint32_t state = h[i].x, count = h[i].y;
        raw = raw && count == (t == 0 ? len : 0u);
        all += count;
        const int r = i % es;  // 4 % es == 0, so t % es == i % es
        if (r < spe) {
            const uint32_t K = len > t ? (len - t + 255) >> 8 : 0;
            const int e = K == z.k[0] ? 0 : K == z.k[1] ? 1 : 2;
            odd = odd || K != z.k[e] || state != z.state[e] || count != z.count[e];
        } else {
            const int g = r - spe;
            odd = odd || state >= 0x80000000u;
            mn[g] = min(mn[g], count);
            mx[g] = max(mx[g], count);
            live += count;
        }
    }
    raw = __all(raw) && len > 0;
    odd = __any(odd);
    v.all_bytes = wave_sum(all);
    v.live_bytes = wave_sum(live);
    v.kind = raw ? 1u : odd ? 2u : 0u;
    for (int g = 0; g < es - spe; g++) {
        v.base[g] = wave_min(mn[g]);
        const uint32_t d = wave_max(mx[g]) - v.base[g];
        v.w[g] = d ? 32 - __clz(d) : 0;
    }
    return v;
}

__device__ inline uint64_t record_bytes(const UnitView& v, int es, int spe) {
    if (v.kind == 1) return 1;
    if (v.kind == 2) return 1 + 256 * 8;
    const int G = es - spe;
    const uint32_t per_plane = 256 / es;
    uint64_t bits = 31ull * per_plane * G;
    for (int g = 0; g < G; g++) bits += (uint64_t)per_plane * v.w[g];
    return 1 + 5ull * G + (bits + 7) / 8;
}

__device__ inline uint64_t stored_bytes(const UnitView& v, uint32_t len) {
    return v.kind == 1 ? len : v.kind == 2 ? v.all_bytes : v.live_bytes;
}

__device__ inline void load_headers(const ckr_stream_header* hdr, uint64_t u, uint4 h[4]) {
    const uint4* p = reinterpret_cast<const uint4*>(hdr + u * 256) + 4 * threadIdx.x;
    for (int i = 0; i < 4; i++) h[i] = p[i];
}

__global__ void __launch_bounds__(kThreads) unit_plan_kernel(const ckr_stream_header* __restrict__ hdr,
                                                             UnitGeomArg g, ZeroLaneArg z,
                                                             uint32_t* __restrict__ rec_size,
                                                             uint32_t* __restrict__ data_size) {
    for (uint64_t u = blockIdx.x; u < g.n_units; u += gridDim.x) {
        const uint32_t len = (uint32_t)min<uint64_t>(g.unit, g.n_bytes - u * g.unit);
        uint4 h[4];
        load_headers(hdr, u, h);
        const UnitView v = analyse_unit(h, len, g.es, g.spe, z);
        if (threadIdx.x == 0) {
            rec_size[u] = (uint32_t)record_bytes(v, g.es, g.spe);
            data_size[u] = (uint32_t)stored_bytes(v, len);
        }
    }
}

// Bits [pos, pos + w) of the LDS stream get the low w bits of val (w <= 32).
__device__ inline void put_bits(uint32_t* words, uint64_t pos, uint32_t val, uint32_t w) {
    if (w == 0) return;
    if (w < 32) val &= (1u << w) - 1;
    const uint32_t q = (uint32_t)(pos >> 5), r = (uint32_t)(pos & 31);
    atomicOr(&words[q], val << r);
    if (r + w > 32) atomicOr(&words[q + 1], val >> (32 - r));
}

__global__ void __launch_bounds__(kThreads) unit_pack_kernel(const uint8_t* __restrict__ data,
                                                             const uint64_t* __restrict__ unit_off,
                                                             const ckr_stream_header* __restrict__ hdr,
                                                             UnitGeomArg g, ZeroLaneArg z,
                                                             const uint64_t* __restrict__ rec_off,
                                                             const uint64_t* __restrict__ out_off,
                                                             uint8_t* __restrict__ rec_out,
                                                             uint8_t* __restrict__ data_out) {
    __shared__ uint32_t bits[512];      // 256 * 31 + 256 * 32 bits at most (16128)
    __shared__ uint32_t run_dst[257];   // stored offset of each kept lane (exclusive, in lane order)
    __shared__ uint32_t run_src[256];   // its offset in the unit's data
    const int j = threadIdx.x;
    for (uint64_t u = blockIdx.x; u < g.n_units; u += gridDim.x) {
        const uint32_t len = (uint32_t)min<uint64_t>(g.unit, g.n_bytes - u * g.unit);
        uint4 h[4];
        load_headers(hdr, u, h);
        const UnitView v = analyse_unit(h, len, g.es, g.spe, z);
        const uint8_t* src = data + unit_off[u];
        uint8_t* rec = rec_out + rec_off[u];
        uint8_t* dst = data_out + out_off[u];
        if (v.kind == 1) {
            if (j == 0) rec[0] = 1;
            for (uint32_t p = j; p < len; p += kThreads) dst[p] = src[p];
            continue;
        }
        if (v.kind == 2) {
            if (j == 0) rec[0] = 2;
            for (int i = 0; i < 4; i++) {
                const uint32_t t = 4 * j + i;
                uint8_t* q = rec + 1 + 8 * t;
                for (int b = 0; b < 4; b++) {
                    q[b] = (uint8_t)(h[i].x >> (8 * b));
                    q[4 + b] = (uint8_t)(h[i].y >> (8 * b));
                }
            }
            for (uint32_t p = j; p < v.all_bytes; p += kThreads) dst[p] = src[p];
            continue;
        }
        // packed: header bytes
        const int G = g.es - g.spe;
        if (j < G) {
            uint8_t* q = rec + 1 + 5 * j;
            for (int b = 0; b < 4; b++) q[b] = (uint8_t)(v.base[j] >> (8 * b));
            q[4] = (uint8_t)v.w[j];
        }
        if (j == 0) rec[0] = 0;
        for (int i = j; i < 512; i += kThreads) bits[i] = 0;
        __syncthreads();
        // bit stream: states, then count deltas; kept-lane offsets for the copy
        const uint32_t per_plane = 256 / g.es, n_live = per_plane * G;
        uint32_t wsum = 0, wpre[4];
        for (int q = 0; q < G; q++) { wpre[q] = wsum; wsum += v.w[q]; }
        uint32_t mine = 0;
        for (int i = 0; i < 4; i++) {
            const uint32_t t = 4 * j + i;
            const int r = i % g.es;
            if (r < g.spe) continue;
            const int q = r - g.spe;
            const uint32_t li = (t / g.es) * G + q;  // index among live lanes
            put_bits(bits, 31ull * li, h[i].x, 31);
            put_bits(bits, 31ull * n_live + (uint64_t)(t / g.es) * wsum + wpre[q], h[i].y - v.base[q], v.w[q]);
            mine += h[i].y;
        }
        uint32_t incl = mine;  // inclusive scan of kept bytes over the wave
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = __shfl_up(incl, d, 64);
            if (j >= d) incl += o;
        }
        uint32_t at = incl - mine;
        for (int i = 0; i < 4; i++) {
            const uint32_t t = 4 * j + i;
            if (i % g.es < g.spe) continue;
            const uint32_t li = (t / g.es) * G + (i % g.es - g.spe);
            run_dst[li] = at;
            run_src[li] = h[i].z;  // buf_offset inside the unit
            at += h[i].y;
        }
        if (j == 63) run_dst[n_live] = incl;
        __syncthreads();
        const uint64_t nbits = 31ull * n_live + (uint64_t)per_plane * wsum;
        const uint32_t nbytes = (uint32_t)((nbits + 7) / 8);
        uint8_t* bs = rec + 1 + 5 * G;
        for (uint32_t p = j; p < nbytes; p += kThreads) bs[p] = (uint8_t)(bits[p >> 2] >> (8 * (p & 3)));
        // kept bytes: byte p of the stored run belongs to the last kept lane whose start <= p
        for (uint32_t p = j; p < v.live_bytes; p += kThreads) {
            uint32_t lo = 0, hi = n_live - 1;
            while (lo < hi) {
                const uint32_t mid = (lo + hi + 1) >> 1;
                if (run_dst[mid] <= p) lo = mid; else hi = mid - 1;
            }
            dst[p] = src[run_src[lo] + (p - run_dst[lo])];
        }
        __syncthreads();  // LDS reused by the next unit
    }
}

uint32_t grid_for(uint64_t n_units) { return (uint32_t)std::min<uint64_t>(n_units, 1u << 16); }

}  // namespace

hipError_t launch_unit_plan(const ckr_stream_header* hdr, const UnitGeomArg& g, const ZeroLaneArg& z,
                            uint32_t* rec_size, uint32_t* data_size, hipStream_t s) {
    if (!g.n_units) return hipSuccess;
    CKR_LAUNCH("unit_plan_kernel", s, unit_plan_kernel<<<grid_for(g.n_units), kThreads, 0, s>>>(hdr, g, z, rec_size, data_size));
    return hipGetLastError();
}

hipError_t launch_unit_pack(const uint8_t* data, const uint64_t* unit_off, const ckr_stream_header* hdr,
                            const UnitGeomArg& g, const ZeroLaneArg& z, const uint64_t* rec_off,
                            const uint64_t* out_off, uint8_t* rec_out, uint8_t* data_out, hipStream_t s) {
    if (!g.n_units) return hipSuccess;
    CKR_LAUNCH("unit_pack_kernel", s, unit_pack_kernel<<<grid_for(g.n_units), kThreads, 0, s>>>(data, unit_off, hdr, g, z, rec_off, out_off, rec_out, data_out));
    return hipGetLastError();
}

// The stream of K zero symbols as rans_encode_kernel writes it
// (src/ANSCompressor.cpp:178-203, cum 0; f == 0: each symbol a raw byte).
uint32_t zero_lane_stream(const ckr_freq_table* t, uint32_t K, std::vector<uint8_t>* bytes) {
    const uint32_t f = t->norm_freq[0];
    std::vector<uint8_t> rev;
    uint32_t x = CKR_L;
    for (uint32_t k = 0; k < K; k++) {
        if (f == 0) {
            rev.push_back(0);
            continue;
        }
        while (x >= f * CKR_NORM_BASE) {
            rev.push_back((uint8_t)(x & 255u));
            x >>= 8;
        }
        x = ((x / f) << CKR_SCALE_BITS) + (x % f);
    }
    if (bytes) bytes->assign(rev.rbegin(), rev.rend());  // written backward: last emitted byte first
    return x;
}

ZeroLanes zero_lanes(const ckr_freq_table* t, uint64_t n_bytes, uint64_t unit) {
    ZeroLanes z;
    const uint64_t nu = (n_bytes + unit - 1) / unit;
    const uint64_t last = nu ? n_bytes - (nu - 1) * unit : 0;
    const uint32_t ks[3] = {(uint32_t)((unit + 255) / 256), (uint32_t)((last + 255) / 256), (uint32_t)(last / 256)};
    for (int e = 0; e < 3; e++) {
        z.arg.k[e] = ks[e];
        z.arg.state[e] = zero_lane_stream(t, ks[e], &z.bytes[e]);
        z.arg.count[e] = (uint32_t)z.bytes[e].size();
    }
    return z;
}

namespace {
struct BitReader {
    const uint8_t* p;
    uint64_t nbytes;
    uint32_t get(uint64_t pos, uint32_t w) const {  // w <= 32, pos + w <= 8 * nbytes
        uint64_t v = 0;
        const uint64_t b0 = pos >> 3;
        for (uint64_t b = b0; b < std::min<uint64_t>(b0 + 5, nbytes); b++) v |= (uint64_t)p[b] << (8 * (b - b0));
        v >>= (pos & 7);
        return w == 32 ? (uint32_t)v : (uint32_t)(v & ((1ull << w) - 1));
    }
};
}  // namespace

int expand_units(const uint8_t* rec, uint64_t rec_size, const uint8_t* stored, uint64_t stored_size,
                 uint64_t n_bytes, uint64_t unit, int es, int spe, const ZeroLanes& z,
                 std::vector<ckr_stream_header>& hdr, std::vector<uint64_t>& uoff, std::vector<uint8_t>& data,
                 std::string& why) {
    const uint64_t nu = n_bytes ? (n_bytes + unit - 1) / unit : 0;
    hdr.assign(nu * 256, ckr_stream_header{0, 0, 0, 0});
    uoff.assign(nu + 1, 0);
    data.clear();
    const int G = es - spe;
    const uint32_t per_plane = 256 / es, n_live = per_plane * G;
    uint64_t rp = 0, sp = 0;
    for (uint64_t u = 0; u < nu; u++) {
        const uint32_t len = (uint32_t)std::min<uint64_t>(unit, n_bytes - u * unit);
        ckr_stream_header* h = &hdr[u * 256];
        if (rp >= rec_size) { why = "records end early"; return CKR_E_CORRUPT; }
        const uint8_t kind = rec[rp];
        const uint64_t start = data.size();
        if (kind == 1) {
            rp += 1;
            if (sp + len > stored_size) { why = "stored bytes end early"; return CKR_E_CORRUPT; }
            h[0].byte_count = len;
            data.insert(data.end(), stored + sp, stored + sp + len);
            sp += len;
        } else if (kind == 2) {
            if (rp + 1 + 2048 > rec_size) { why = "records end early"; return CKR_E_CORRUPT; }
            uint64_t all = 0;
            for (int t = 0; t < 256; t++) {
                std::memcpy(&h[t].final_state, rec + rp + 1 + 8 * t, 4);
                std::memcpy(&h[t].byte_count, rec + rp + 5 + 8 * t, 4);
                all += h[t].byte_count;
            }
            rp += 1 + 2048;
            if (all > len || sp + all > stored_size) { why = "unit bytes out of range"; return CKR_E_CORRUPT; }
            data.insert(data.end(), stored + sp, stored + sp + all);
            sp += all;
        } else if (kind == 0) {
            if (rp + 1 + 5ull * G > rec_size) { why = "records end early"; return CKR_E_CORRUPT; }
            uint32_t base[4], w[4], wpre[4], wsum = 0;
            for (int q = 0; q < G; q++) {
                std::memcpy(&base[q], rec + rp + 1 + 5 * q, 4);
                w[q] = rec[rp + 5 + 5 * q];
                if (w[q] > 32) { why = "bit width above 32"; return CKR_E_CORRUPT; }
                wpre[q] = wsum;
                wsum += w[q];
            }
            const uint64_t nbits = 31ull * n_live + (uint64_t)per_plane * wsum;
            const uint64_t nb = (nbits + 7) / 8;
            const uint64_t bs = rp + 1 + 5ull * G;
            if (bs + nb > rec_size) { why = "records end early"; return CKR_E_CORRUPT; }
            const BitReader br{rec + bs, nb};
            uint64_t live = 0;
            for (uint32_t t = 0; t < 256; t++) {
                const int r = (int)(t % es);
                if (r < spe) continue;
                const int q = r - spe;
                const uint32_t li = (t / es) * G + q;
                h[t].final_state = br.get(31ull * li, 31);
                const uint64_t c = (uint64_t)base[q] + br.get(31ull * n_live + (uint64_t)(t / es) * wsum + wpre[q], w[q]);
                if (c > 0xFFFFFFFFull) { why = "byte count above 32 bits"; return CKR_E_CORRUPT; }
                h[t].byte_count = (uint32_t)c;
                live += c;
            }
            rp = bs + nb;
            if (live > len || sp + live > stored_size) { why = "unit bytes out of range"; return CKR_E_CORRUPT; }
            // lanes in order: kept bytes from the stored run, zero-plane lanes from their K
            for (uint32_t t = 0; t < 256; t++) {
                if ((int)(t % es) < spe) {
                    const uint32_t K = len > t ? (len - t + 255) / 256 : 0;
                    const int e = K == z.arg.k[0] ? 0 : K == z.arg.k[1] ? 1 : 2;
                    h[t].final_state = z.arg.state[e];
                    h[t].byte_count = z.arg.count[e];
                    data.insert(data.end(), z.bytes[e].begin(), z.bytes[e].end());
                } else {
                    data.insert(data.end(), stored + sp, stored + sp + h[t].byte_count);
                    sp += h[t].byte_count;
                }
            }
        } else {
            why = "unknown unit kind";
            return CKR_E_CORRUPT;
        }
        if (kind != 1) {
            uint32_t off = 0;
            for (int t = 0; t < 256; t++) { h[t].buf_offset = off; off += h[t].byte_count; }
        }
        uoff[u + 1] = uoff[u] + (data.size() - start);
    }
    if (rp != rec_size || sp != stored_size) { why = "records or stored bytes left over"; return CKR_E_CORRUPT; }
    return CKR_OK;
}

}  // namespace ckr
