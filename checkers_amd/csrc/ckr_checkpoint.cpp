// checkers_amd/csrc/ckr_checkpoint.cpp — rank checkpoint files around the GPU
// codec: fingerprint weights and clusters (host), the compress-and-save
// orchestration, the .ansc / .mant / .dict writers, and a reader that restores
// tensors on the device.
//
// Reference (paths relative to the reference tree):
//   TensorAnalyzer::compute_fingerprint_weights   src/TensorAnalyzer.cpp:322-380
//   TensorAnalyzer::build_knn_clusters            src/TensorAnalyzer.cpp:440-598
//   ANSCompressor::compress_and_save_all          src/ANSCompressor.cpp:1014-1401
//   write_rank_states_file / _mantissa_ / _tables_ src/ANSCompressor.cpp:721-931
// The reference has no reader; ckr_ckpt_open / ckr_ckpt_restore are this
// library's own, over the same formats.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <map>
#include <numeric>
#include <string>
#include <unordered_map>
#include <vector>

#include "checkers_amd.h"
#include "ckr_internal.h"

namespace {

namespace fs = std::filesystem;

constexpr uint32_t kAnscMagic = 0x414E5343u;  // "ANSC"
constexpr uint32_t kMantMagic = 0x4D414E54u;  // "MANT"
constexpr uint32_t kDictMagic = 0x44494354u;  // "DICT"
constexpr uint64_t kV2Entry = 256 + 8 + 32 + 256 + 256 * 16;  // 4648
constexpr uint64_t kV3Entry = 256 + 8 + 32 + 256 + 16;        // 568
constexpr uint64_t kMantEntry = 288;
constexpr uint64_t kDictEntry = 2308;

int err(int code, const std::string& m) { return ckr::set_error(code, m); }

#define CKP_HIP(call)                                                                                    \
    do {                                                                                                 \
        hipError_t _e = (call);                                                                          \
        if (_e != hipSuccess) return err(CKR_E_HIP, std::string("[ckr] HIP error in " #call ": ") + hipGetErrorString(_e)); \
    } while (0)

// ---- fingerprint weights and clusters

// Category of a record by its name prefix (build_knn_clusters, :452-457).
std::string category_of(const std::string& name) {
    auto starts = [&](const char* p) { return name.rfind(p, 0) == 0; };
    if (starts("optimizer.exp_avg_sq::")) return "exp_avg_sq";
    if (starts("optimizer.exp_avg::")) return "exp_avg";
    if (starts("master_weights::")) return "master_weights";
    return "model_state";
}

// Union-find with path compression and union by rank.  Which element ends up
// as a root decides the order in which clusters are numbered, so the merge rule
// is fixed: the root of higher rank wins, on equal rank the first argument's.
struct DisjointSets {
    std::vector<int> parent, rank;
    explicit DisjointSets(int n) : parent(n), rank(n, 0) { std::iota(parent.begin(), parent.end(), 0); }
    int root(int x) { return parent[x] == x ? x : parent[x] = root(parent[x]); }
    void join(int a, int b) {
        a = root(a);
        b = root(b);
        if (a == b) return;
        if (rank[a] < rank[b]) std::swap(a, b);
        parent[b] = a;
        if (rank[a] == rank[b]) rank[a]++;
    }
};

// ---- little-endian file helpers
struct Out {
    std::ofstream f;
    explicit Out(const fs::path& p) : f(p, std::ios::binary | std::ios::trunc) {}
    void put(const void* p, size_t n) { f.write(static_cast<const char*>(p), (std::streamsize)n); }
    void u8(uint8_t v) { put(&v, 1); }
    void u32(uint32_t v) { put(&v, 4); }
    void u64(uint64_t v) { put(&v, 8); }
    void zeros(size_t n) { static const char z[64] = {}; while (n) { size_t k = std::min<size_t>(n, 64); put(z, k); n -= k; } }
    void name(const std::string& s) {  // 256 bytes, at most 255 copied, NUL padded
        char b[256] = {};
        std::memcpy(b, s.data(), std::min<size_t>(s.size(), 255));
        put(b, 256);
    }
};

struct TensorOut {
    std::string name, anchor;
    int dtype = 0;
    bool owns = false;
    uint64_t n_elems = 0, original = 0;
    std::vector<uint8_t> data, sidecar;
    std::vector<ckr_stream_header> headers;  // n_units * 256
    std::vector<uint64_t> unit_off;          // n_units + 1
    uint32_t spe = 0;
    ckr_freq_table* table = nullptr;         // owners: the table they built
};

bool unit_is_raw(const ckr_stream_header* h, uint64_t len) {
    if (h[0].byte_count != (uint32_t)len) return false;
    for (int t = 1; t < 256; t++)
        if (h[t].byte_count) return false;
    return true;
}

int write_files(const fs::path& dir, int rank, uint64_t unit_bytes, const std::vector<TensorOut>& ts) {
    std::error_code ec;
    fs::create_directories(dir / "mantissa", ec);
    fs::create_directories(dir / "tables", ec);
    if (ec) return err(CKR_E_INVALID, "[ckr] cannot create " + dir.string() + ": " + ec.message());
    const uint32_t r = (uint32_t)(rank < 0 ? 0 : rank);
    const std::string tag = "rank_" + std::to_string(rank < 0 ? 0 : rank);
    {
        const fs::path p = dir / (tag + "_states.ansc");
        Out o(p);
        if (!o.f) return err(CKR_E_INVALID, "[ANS] cannot open for write: " + p.string());
        const bool v3 = unit_bytes != 0;
        o.u32(kAnscMagic);
        o.u32(v3 ? 3u : 2u);
        o.u32(r);
        o.u32((uint32_t)ts.size());
        if (v3) o.u64(unit_bytes);
        // per-unit metadata section of v3: headers then unit offsets, tensor after tensor
        std::vector<uint64_t> meta_off(ts.size() + 1, 0);
        for (size_t i = 0; i < ts.size(); i++)
            meta_off[i + 1] = meta_off[i] + ts[i].headers.size() * 16 + ts[i].unit_off.size() * 8;
        uint64_t doff = 0;
        for (const auto& t : ts) {
            o.name(t.name);
            const uint64_t nu = t.unit_off.empty() ? 0 : t.unit_off.size() - 1;
            bool raw = nu > 0;
            for (uint64_t u = 0; u < nu && raw; u++) {
                const uint64_t len = v3 ? std::min<uint64_t>(unit_bytes, t.original - u * unit_bytes) : t.original;
                raw = unit_is_raw(&t.headers[u * 256], len);
            }
            o.u8((uint8_t)t.dtype);
            o.u8(raw ? 1 : 0);
            o.u8(t.owns ? 1 : 0);
            o.zeros(5);
            o.u64(t.original);
            o.u64(t.n_elems);
            o.u64(doff);
            o.u64(t.data.size());
            doff += t.data.size();
            o.name(t.owns ? std::string() : t.anchor);
            if (v3) {
                o.u64(nu);
                o.u64(meta_off[&t - ts.data()]);
            } else {
                o.put(t.headers.data(), 256 * 16);
            }
        }
        if (v3)
            for (const auto& t : ts) {
                o.put(t.headers.data(), t.headers.size() * 16);
                o.put(t.unit_off.data(), t.unit_off.size() * 8);
            }
        for (const auto& t : ts) o.put(t.data.data(), t.data.size());
        if (!o.f) return err(CKR_E_INVALID, "[ckr] write failed: " + p.string());
    }
    {
        const fs::path p = dir / "mantissa" / (tag + "_mantissa.mant");
        Out o(p);
        if (!o.f) return err(CKR_E_INVALID, "[ANS] cannot open mantissa for write: " + p.string());
        uint32_t cnt = 0;
        for (const auto& t : ts) cnt += t.spe > 0;
        o.u32(kMantMagic);
        o.u32(2u);
        o.u32(r);
        o.u32(cnt);
        uint64_t doff = 0;
        for (const auto& t : ts) {
            if (!t.spe) continue;
            o.name(t.name);
            o.u8((uint8_t)t.dtype);
            o.u8((uint8_t)t.spe);
            o.zeros(6);
            o.u64(t.n_elems);
            o.u64(doff);
            o.u64(t.sidecar.size());
            doff += t.sidecar.size();
        }
        for (const auto& t : ts)
            if (t.spe) o.put(t.sidecar.data(), t.sidecar.size());
        if (!o.f) return err(CKR_E_INVALID, "[ckr] write failed: " + p.string());
    }
    {
        const fs::path p = dir / "tables" / (tag + "_tables.dict");
        Out o(p);
        if (!o.f) return err(CKR_E_INVALID, "[ANS] cannot open tables for write: " + p.string());
        uint32_t cnt = 0;
        for (const auto& t : ts) cnt += t.owns;
        o.u32(kDictMagic);
        o.u32(1u);
        o.u32(r);
        o.u32(cnt);
        for (const auto& t : ts) {
            if (!t.owns) continue;
            o.name(t.name);
            o.put(t.table->norm_freq, 256 * 4);
            o.put(t.table->cum_freq, 257 * 4);
        }
        if (!o.f) return err(CKR_E_INVALID, "[ckr] write failed: " + p.string());
    }
    return CKR_OK;
}

// Table from stored norm/cum (the decode arrays are rebuilt by the decoder).
void table_from_norm(const uint32_t* norm, const uint32_t* cum, ckr_freq_table* t) {
    std::memset(t, 0, sizeof(*t));
    std::memcpy(t->norm_freq, norm, 256 * 4);
    std::memcpy(t->cum_freq, cum, 257 * 4);
    for (int s = 0; s < 256; s++) t->x_max[s] = CKR_NORM_BASE * norm[s];
}

// Largest-first decrements until the table sums to M (only for a table the
// reference's one-pass correction left above M).
void repair_table(ckr_freq_table* t) {
    uint32_t sum = 0;
    for (int s = 0; s < 256; s++) sum += t->norm_freq[s];
    while (sum > CKR_M) {
        int best = -1;
        for (int s = 0; s < 256; s++)
            if (t->norm_freq[s] > 1 && (best < 0 || t->norm_freq[s] > t->norm_freq[best])) best = s;
        if (best < 0) break;
        t->norm_freq[best]--;
        sum--;
    }
    uint32_t c = 0;
    for (int s = 0; s < 256; s++) { t->cum_freq[s] = c; c += t->norm_freq[s]; t->x_max[s] = CKR_NORM_BASE * t->norm_freq[s]; }
    t->cum_freq[256] = c;
}

}  // namespace

// ---------------------------------------------------------------- reader state
struct ckr_ckpt {
    fs::path dir;
    uint32_t version = 0, rank = 0;
    uint64_t unit_bytes = 0;
    struct Entry {
        std::string name, anchor;
        uint8_t dtype = 0, raw = 0, owns = 0;
        uint64_t original = 0, n_elems = 0, data_off = 0, data_size = 0, n_units = 0, meta_off = 0;
        std::vector<ckr_stream_header> v2_headers;
    };
    std::vector<Entry> entries;
    uint64_t meta_base = 0, data_base = 0;
    struct Side { uint8_t dtype = 0, bpe = 0; uint64_t n = 0, off = 0, size = 0; };
    std::map<std::string, Side> sidecars;
    uint64_t mant_data_base = 0;
    std::map<std::string, std::pair<std::vector<uint32_t>, std::vector<uint32_t>>> tables;
};

extern "C" {

int ckr_fingerprint_weights(const float* h_fp, uint64_t n, double* h_weights) {
    if ((n && !h_fp) || !h_weights) return err(CKR_E_INVALID, "[ckr] null pointer");
    // compute_fingerprint_weights (TensorAnalyzer.cpp:322-380): per-dimension
    // variance over all records, normalised by sum(variance + 1e-8)
    double m[5] = {}, m2[5] = {};
    for (uint64_t i = 0; i < n; i++)
        for (int d = 0; d < 5; d++) {
            const double v = (double)h_fp[5 * i + d];
            m[d] += v;
            m2[d] += v * v;
        }
    double imp[5], sum = 0.0;
    for (int d = 0; d < 5; d++) {
        imp[d] = n ? m2[d] / (double)n - (m[d] / (double)n) * (m[d] / (double)n) : 0.0;
        sum += imp[d] + 1e-8;
    }
    for (int d = 0; d < 5; d++) h_weights[d] = imp[d] / sum;
    return CKR_OK;
}

int ckr_cluster(const char* const* names, const float* h_fp, uint64_t n, int32_t* h_cluster_of, double* h_threshold) {
    if (n && (!names || !h_fp || !h_cluster_of)) return err(CKR_E_INVALID, "[ckr] null pointer");
    std::map<std::string, std::vector<uint64_t>> by_cat;
    for (uint64_t i = 0; i < n; i++) by_cat[category_of(names[i] ? names[i] : "")].push_back(i);
    int32_t next_id = 0;
    int ci = 0;
    for (const auto& kv : by_cat) {
        const std::vector<uint64_t>& idx = kv.second;
        const int k = (int)idx.size();
        double mean[5] = {}, sd[5] = {};
        for (int a = 0; a < k; a++)
            for (int d = 0; d < 5; d++) mean[d] += (double)h_fp[5 * idx[a] + d];
        for (int d = 0; d < 5; d++) mean[d] /= k;
        for (int a = 0; a < k; a++)
            for (int d = 0; d < 5; d++) {
                const double x = (double)h_fp[5 * idx[a] + d] - mean[d];
                sd[d] += x * x;
            }
        for (int d = 0; d < 5; d++) sd[d] = (sd[d] / k < 1e-30) ? 1.0 : std::sqrt(sd[d] / k);
        auto dist = [&](int a, int b) {
            double s = 0;
            for (int d = 0; d < 5; d++) {
                const double x = ((double)h_fp[5 * idx[a] + d] - (double)h_fp[5 * idx[b] + d]) / sd[d];
                s += x * x;
            }
            return std::sqrt(s);
        };
        std::vector<double> all;
        all.reserve((size_t)k * (k - 1) / 2);
        for (int a = 0; a < k; a++)
            for (int b = a + 1; b < k; b++) all.push_back(dist(a, b));
        double thr = 0.0;
        if (!all.empty()) {
            std::sort(all.begin(), all.end());
            thr = all[all.size() / 4];  // lower quartile
        }
        if (h_threshold) h_threshold[ci] = thr;
        ci++;
        DisjointSets ds(k);
        for (int a = 0; a < k; a++)
            for (int b = a + 1; b < k; b++)
                if (dist(a, b) < thr) ds.join(a, b);
        std::map<int, std::vector<int>> groups;  // root → members in order
        for (int a = 0; a < k; a++) groups[ds.root(a)].push_back(a);
        for (const auto& [root, mem] : groups) {
            if (mem.size() >= 2) {
                for (int a : mem) h_cluster_of[idx[a]] = next_id;
                next_id++;
            } else {
                h_cluster_of[idx[mem[0]]] = -1;
            }
        }
    }
    return CKR_OK;
}

int ckr_ckpt_write(const char* output_dir, int rank, const ckr_ckpt_tensor* tensors, uint64_t n, uint64_t unit_bytes,
                   int repair_tables, ckr_ckpt_stats* h_stats, void* stream) {
    if (!output_dir || (n && !tensors)) return err(CKR_E_INVALID, "[ckr] null pointer");
    if (unit_bytes % 256) return err(CKR_E_INVALID, "[ckr] unit_bytes must be a multiple of 256");
    hipStream_t s = (hipStream_t)stream;
    // anchors: the first record of each cluster (cluster_anchor); the table
    // owner is the first one that is compressed (compress_and_save_all :1057-1069)
    std::unordered_map<int32_t, std::string> anchor_name;
    for (uint64_t i = 0; i < n; i++)
        if (tensors[i].cluster_id >= 0 && !anchor_name.count(tensors[i].cluster_id))
            anchor_name[tensors[i].cluster_id] = tensors[i].name ? tensors[i].name : "";
    std::unordered_map<int32_t, ckr_freq_table*> cluster_table;
    std::vector<TensorOut> outs;
    std::vector<ckr_freq_table> tables(n);
    outs.reserve(n);
    uint64_t cap_ws = 0, cap_out = 0, cap_hdr = 0, cap_off = 0, cap_side = 0;
    for (uint64_t i = 0; i < n; i++) {
        const auto& t = tensors[i];
        if (!t.d_ptr || !t.num_elements) continue;
        const int es = ckr_element_size(t.dtype);
        if (!es) return err(CKR_E_INVALID, "[ckr] unknown dtype for tensor " + std::string(t.name ? t.name : ""));
        const uint64_t nu = ckr_num_units(t.num_elements, t.dtype, unit_bytes);
        if (!unit_bytes && t.num_elements * es > 0xFFFFFFFFull)
            return err(CKR_E_INVALID, "[ckr] tensor " + std::string(t.name) + " needs unit_bytes (over 4 GiB)");
        cap_ws = std::max(cap_ws, ckr_encode_workspace_bytes(t.num_elements, t.dtype, unit_bytes));
        cap_out = std::max(cap_out, t.num_elements * es);
        cap_hdr = std::max(cap_hdr, nu * 256 * 16);
        cap_off = std::max(cap_off, (nu + 1) * 8);
        cap_side = std::max(cap_side, t.num_elements * (uint64_t)ckr_sidecar_bytes_per_elem(t.dtype));
    }
    void *d_ws = nullptr, *d_out = nullptr, *d_hdr = nullptr, *d_off = nullptr, *d_side = nullptr;
    auto release = [&]() {
        for (void* p : {d_ws, d_out, d_hdr, d_off, d_side}) if (p) (void)hipFree(p);
    };
    auto alloc = [&](void** p, uint64_t b) { return hipMalloc(p, std::max<uint64_t>(b, 256)); };
    if (cap_out == 0) return write_files(fs::path(output_dir), rank, unit_bytes, outs);  // nothing to compress
    if (alloc(&d_ws, cap_ws) != hipSuccess || alloc(&d_out, cap_out) != hipSuccess ||
        alloc(&d_hdr, cap_hdr) != hipSuccess || alloc(&d_off, cap_off) != hipSuccess ||
        alloc(&d_side, cap_side) != hipSuccess) {
        release();
        return err(CKR_E_HIP, "[ckr] device allocation for the checkpoint writer failed");
    }
    int rc = CKR_OK;
    uint64_t si = 0;
    for (uint64_t i = 0; i < n && rc == CKR_OK; i++) {
        const auto& t = tensors[i];
        if (!t.d_ptr || !t.num_elements) continue;
        TensorOut o;
        o.name = t.name ? t.name : "";
        o.dtype = t.dtype;
        o.n_elems = t.num_elements;
        o.original = t.num_elements * (uint64_t)ckr_element_size(t.dtype);
        o.spe = (uint32_t)ckr_sidecar_bytes_per_elem(t.dtype);
        const bool singleton = t.cluster_id < 0;
        auto it = cluster_table.find(t.cluster_id);
        o.owns = singleton || it == cluster_table.end();
        ckr_freq_table* tab = &tables[i];
        const uint64_t ws = ckr_encode_workspace_bytes(t.num_elements, t.dtype, unit_bytes);
        uint64_t total = 0;
        uint32_t tsum = CKR_M;
        if (o.owns) {
            rc = ckr_compress(t.d_ptr, t.num_elements, t.dtype, unit_bytes, singleton ? 0 : 1, (uint8_t*)d_out, cap_out,
                              (ckr_stream_header*)d_hdr, (uint64_t*)d_off, (uint8_t*)d_side, d_ws, ws, tab, &total, s);
            tsum = tab->cum_freq[256];
            if (rc == CKR_OK && repair_tables && tsum > CKR_M) {
                repair_table(tab);
                rc = ckr_encode(t.d_ptr, t.num_elements, t.dtype, tab, unit_bytes, (uint8_t*)d_out, cap_out,
                                (ckr_stream_header*)d_hdr, (uint64_t*)d_off, (uint8_t*)d_side, d_ws, ws, &total, s);
            }
            if (!singleton) cluster_table[t.cluster_id] = tab;
            o.table = tab;
        } else {
            tab = it->second;
            tsum = tab->cum_freq[256];
            o.anchor = anchor_name[t.cluster_id];
            rc = ckr_encode(t.d_ptr, t.num_elements, t.dtype, tab, unit_bytes, (uint8_t*)d_out, cap_out,
                            (ckr_stream_header*)d_hdr, (uint64_t*)d_off, (uint8_t*)d_side, d_ws, ws, &total, s);
        }
        if (rc != CKR_OK) break;
        const uint64_t nu = ckr_num_units(t.num_elements, t.dtype, unit_bytes);
        o.data.resize(total);
        o.headers.resize(nu * 256);
        o.unit_off.resize(nu + 1);
        o.sidecar.resize(t.num_elements * o.spe);
        if (total && hipMemcpyAsync(o.data.data(), d_out, total, hipMemcpyDeviceToHost, s) != hipSuccess) rc = CKR_E_HIP;
        if (hipMemcpyAsync(o.headers.data(), d_hdr, nu * 256 * 16, hipMemcpyDeviceToHost, s) != hipSuccess) rc = CKR_E_HIP;
        if (hipMemcpyAsync(o.unit_off.data(), d_off, (nu + 1) * 8, hipMemcpyDeviceToHost, s) != hipSuccess) rc = CKR_E_HIP;
        if (o.spe && hipMemcpyAsync(o.sidecar.data(), d_side, o.sidecar.size(), hipMemcpyDeviceToHost, s) != hipSuccess)
            rc = CKR_E_HIP;
        if (hipStreamSynchronize(s) != hipSuccess) rc = CKR_E_HIP;
        if (rc != CKR_OK) { err(rc, "[ckr] copy of compressed tensor failed"); break; }
        if (h_stats) {
            ckr_ckpt_stats& st = h_stats[si];
            st.record_index = i;
            st.original_bytes = o.original;
            st.ans_bytes = total;
            st.sidecar_bytes = o.sidecar.size();
            st.owns_table = o.owns;
            st.table_sum = tsum;
            st.table_repaired = (o.owns && repair_tables && tsum > CKR_M) ? 1 : 0;
        }
        si++;
        outs.push_back(std::move(o));
    }
    release();
    if (rc != CKR_OK) return rc;
    return write_files(fs::path(output_dir), rank, unit_bytes, outs);
}

}  // extern "C"

// ---------------------------------------------------------------- reader
namespace {
bool read_at(std::ifstream& f, uint64_t off, void* p, uint64_t n) {
    f.clear();
    f.seekg((std::streamoff)off);
    f.read(static_cast<char*>(p), (std::streamsize)n);
    return (uint64_t)f.gcount() == n;
}
std::string cstr(const char* b) { return std::string(b, strnlen(b, 256)); }
// Unit offsets and lane headers read from a file, checked on the host before
// anything reaches the device (the decoders take them as an encode wrote them):
// offsets start at 0, never decrease and end at the data size; no unit is
// longer than its input bytes (the passthrough rule bounds every unit by its
// length); a raw unit is exactly its length with only header 0 set; every
// lane's stream lies inside its unit.
int check_unit_metadata(const std::vector<ckr_stream_header>& hdr, const std::vector<uint64_t>& uoff, uint64_t nu,
                        uint64_t n_bytes, uint64_t unit, uint64_t data_size, const std::string& name) {
    const std::string what = "[ckr] corrupt unit metadata for " + name + ": ";
    if (uoff.size() != nu + 1 || hdr.size() != nu * 256) return err(CKR_E_CORRUPT, what + "sizes");
    if (uoff[0] != 0) return err(CKR_E_CORRUPT, what + "first unit offset is not 0");
    if (uoff[nu] != data_size) return err(CKR_E_CORRUPT, what + "last unit offset is not the data size");
    for (uint64_t u = 0; u < nu; u++) {
        if (uoff[u + 1] < uoff[u]) return err(CKR_E_CORRUPT, what + "unit offsets decrease at unit " + std::to_string(u));
        const uint64_t size = uoff[u + 1] - uoff[u];
        const uint64_t len = std::min<uint64_t>(unit, n_bytes - u * unit);
        if (size > len) return err(CKR_E_CORRUPT, what + "unit " + std::to_string(u) + " is longer than its input");
        const ckr_stream_header* h = &hdr[u * 256];
        if (size == len && h[0].byte_count == len) {
            for (int t = 1; t < 256; t++)
                if (h[t].byte_count) return err(CKR_E_CORRUPT, what + "raw unit " + std::to_string(u) + " has lane bytes");
            continue;
        }
        for (int t = 0; t < 256; t++)
            if ((uint64_t)h[t].buf_offset + h[t].byte_count > size)
                return err(CKR_E_CORRUPT, what + "lane " + std::to_string(t) + " of unit " + std::to_string(u) +
                                              " runs past its unit");
    }
    return CKR_OK;
}
}  // namespace

extern "C" {

int ckr_ckpt_open(const char* dir, int rank, ckr_ckpt** out) {
    if (!dir || !out) return err(CKR_E_INVALID, "[ckr] null pointer");
    *out = nullptr;
    auto c = std::make_unique<ckr_ckpt>();
    c->dir = dir;
    const std::string tag = "rank_" + std::to_string(rank < 0 ? 0 : rank);
    const fs::path sp = c->dir / (tag + "_states.ansc");
    std::ifstream f(sp, std::ios::binary);
    if (!f) return err(CKR_E_INVALID, "[ckr] cannot open " + sp.string());
    uint32_t h[4];
    if (!read_at(f, 0, h, 16) || h[0] != kAnscMagic || (h[1] != 2 && h[1] != 3))
        return err(CKR_E_CORRUPT, "[ckr] not an .ansc v2/v3 file: " + sp.string());
    c->version = h[1];
    c->rank = h[2];
    const uint32_t nt = h[3];
    uint64_t pos = 16;
    if (c->version == 3) {
        if (!read_at(f, 16, &c->unit_bytes, 8)) return err(CKR_E_CORRUPT, "[ckr] truncated header");
        pos = 24;
    }
    const uint64_t esz = c->version == 3 ? kV3Entry : kV2Entry;
    std::vector<uint8_t> buf(esz);
    uint64_t meta_total = 0;
    for (uint32_t i = 0; i < nt; i++, pos += esz) {
        if (!read_at(f, pos, buf.data(), esz)) return err(CKR_E_CORRUPT, "[ckr] truncated index");
        ckr_ckpt::Entry e;
        const uint8_t* b = buf.data();
        e.name = cstr(reinterpret_cast<const char*>(b));
        e.dtype = b[256];
        e.raw = b[257];
        e.owns = b[258];
        std::memcpy(&e.original, b + 264, 8);
        std::memcpy(&e.n_elems, b + 272, 8);
        std::memcpy(&e.data_off, b + 280, 8);
        std::memcpy(&e.data_size, b + 288, 8);
        e.anchor = cstr(reinterpret_cast<const char*>(b + 296));
        if (c->version == 3) {
            std::memcpy(&e.n_units, b + 552, 8);
            std::memcpy(&e.meta_off, b + 560, 8);
            meta_total += e.n_units * 256 * 16 + (e.n_units + 1) * 8;
        } else {
            e.n_units = 1;
            e.v2_headers.resize(256);
            std::memcpy(e.v2_headers.data(), b + 552, 256 * 16);
        }
        c->entries.push_back(std::move(e));
    }
    c->meta_base = pos;
    c->data_base = pos + meta_total;
    // sidecars
    const fs::path mp = c->dir / "mantissa" / (tag + "_mantissa.mant");
    std::ifstream m(mp, std::ios::binary);
    if (m) {
        if (!read_at(m, 0, h, 16) || h[0] != kMantMagic || h[1] != 2)
            return err(CKR_E_CORRUPT, "[ckr] not a .mant v2 file: " + mp.string());
        std::vector<uint8_t> eb(kMantEntry);
        for (uint32_t i = 0; i < h[3]; i++) {
            if (!read_at(m, 16 + i * kMantEntry, eb.data(), kMantEntry)) return err(CKR_E_CORRUPT, "[ckr] truncated .mant");
            ckr_ckpt::Side sd;
            sd.dtype = eb[256];
            sd.bpe = eb[257];
            std::memcpy(&sd.n, eb.data() + 264, 8);
            std::memcpy(&sd.off, eb.data() + 272, 8);
            std::memcpy(&sd.size, eb.data() + 280, 8);
            c->sidecars[cstr(reinterpret_cast<const char*>(eb.data()))] = sd;
        }
        c->mant_data_base = 16 + (uint64_t)h[3] * kMantEntry;
    }
    // tables
    const fs::path dp = c->dir / "tables" / (tag + "_tables.dict");
    std::ifstream d(dp, std::ios::binary);
    if (d) {
        if (!read_at(d, 0, h, 16) || h[0] != kDictMagic || h[1] != 1)
            return err(CKR_E_CORRUPT, "[ckr] not a .dict v1 file: " + dp.string());
        std::vector<uint8_t> eb(kDictEntry);
        for (uint32_t i = 0; i < h[3]; i++) {
            if (!read_at(d, 16 + i * kDictEntry, eb.data(), kDictEntry)) return err(CKR_E_CORRUPT, "[ckr] truncated .dict");
            std::vector<uint32_t> norm(256), cum(257);
            std::memcpy(norm.data(), eb.data() + 256, 1024);
            std::memcpy(cum.data(), eb.data() + 1280, 1028);
            c->tables[cstr(reinterpret_cast<const char*>(eb.data()))] = {norm, cum};
        }
    }
    *out = c.release();
    return CKR_OK;
}

void ckr_ckpt_close(ckr_ckpt* c) { delete c; }

uint64_t ckr_ckpt_count(const ckr_ckpt* c) { return c ? c->entries.size() : 0; }

int ckr_ckpt_info(const ckr_ckpt* c, uint64_t i, ckr_ckpt_entry* e) {
    if (!c || !e || i >= c->entries.size()) return err(CKR_E_INVALID, "[ckr] bad checkpoint entry");
    const auto& x = c->entries[i];
    std::memset(e, 0, sizeof(*e));
    std::memcpy(e->name, x.name.data(), std::min<size_t>(x.name.size(), 255));
    std::memcpy(e->anchor_name, x.anchor.data(), std::min<size_t>(x.anchor.size(), 255));
    e->dtype = x.dtype;
    e->is_raw = x.raw;
    e->owns_table = x.owns;
    e->version = c->version;
    e->original_bytes = x.original;
    e->num_elements = x.n_elems;
    e->data_size = x.data_size;
    e->n_units = x.n_units;
    e->unit_bytes = c->version == 3 ? c->unit_bytes : 0;
    const auto s = c->sidecars.find(x.name);
    e->sidecar_bytes = s == c->sidecars.end() ? 0 : s->second.size;
    return CKR_OK;
}

int ckr_ckpt_restore(const ckr_ckpt* c, uint64_t i, void* d_dst, void* stream) {
    if (!c || i >= c->entries.size() || !d_dst) return err(CKR_E_INVALID, "[ckr] bad restore arguments");
    const auto& x = c->entries[i];
    hipStream_t s = (hipStream_t)stream;
    const int es = ckr_element_size(x.dtype);
    const uint32_t spe = (uint32_t)ckr_sidecar_bytes_per_elem(x.dtype);
    if (!es || x.original != x.n_elems * (uint64_t)es) return err(CKR_E_CORRUPT, "[ckr] inconsistent entry " + x.name);
    const auto tit = c->tables.find(x.owns ? x.name : x.anchor);
    if (tit == c->tables.end()) return err(CKR_E_CORRUPT, "[ckr] no table for " + x.name);
    ckr_freq_table tab;
    table_from_norm(tit->second.first.data(), tit->second.second.data(), &tab);
    const uint64_t unit = c->version == 3 ? c->unit_bytes : 0;
    const uint64_t nu = ckr_num_units(x.n_elems, x.dtype, unit);
    if (nu != x.n_units) return err(CKR_E_CORRUPT, "[ckr] unit count mismatch for " + x.name);
    const fs::path sp = c->dir / ("rank_" + std::to_string(c->rank) + "_states.ansc");
    std::error_code fec;
    const uint64_t fsize = fs::file_size(sp, fec);
    if (fec || nu > fsize / 4096 + 1 || x.data_size > fsize)
        return err(CKR_E_CORRUPT, "[ckr] entry " + x.name + " does not fit its file");
    std::ifstream f(sp, std::ios::binary);
    std::vector<ckr_stream_header> hdr(nu * 256);
    std::vector<uint64_t> uoff(nu + 1);
    if (c->version == 3) {
        if (!read_at(f, c->meta_base + x.meta_off, hdr.data(), hdr.size() * 16) ||
            !read_at(f, c->meta_base + x.meta_off + hdr.size() * 16, uoff.data(), uoff.size() * 8))
            return err(CKR_E_CORRUPT, "[ckr] truncated unit metadata for " + x.name);
    } else {
        hdr = x.v2_headers;
        uoff[0] = 0;
        uoff[1] = x.data_size;
    }
    if (int rc = check_unit_metadata(hdr, uoff, nu, x.original, unit ? unit : x.original, x.data_size, x.name))
        return rc;
    std::vector<uint8_t> data(std::max<uint64_t>(x.data_size, 1));
    if (x.data_size && !read_at(f, c->data_base + x.data_off, data.data(), x.data_size))
        return err(CKR_E_CORRUPT, "[ckr] truncated data for " + x.name);
    std::vector<uint8_t> side;
    if (spe) {
        const auto sit = c->sidecars.find(x.name);
        if (sit == c->sidecars.end() || sit->second.size != x.n_elems * spe)
            return err(CKR_E_CORRUPT, "[ckr] missing sidecar for " + x.name);
        std::ifstream m(c->dir / "mantissa" / ("rank_" + std::to_string(c->rank) + "_mantissa.mant"), std::ios::binary);
        side.resize(sit->second.size);
        if (!read_at(m, c->mant_data_base + sit->second.off, side.data(), side.size()))
            return err(CKR_E_CORRUPT, "[ckr] truncated sidecar for " + x.name);
    }
    const uint64_t wsb = ckr_decode_workspace_bytes(x.n_elems, x.dtype, unit);
    void *d_data = nullptr, *d_hdr = nullptr, *d_off = nullptr, *d_side = nullptr, *d_ws = nullptr;
    auto release = [&]() { for (void* p : {d_data, d_hdr, d_off, d_side, d_ws}) if (p) (void)hipFree(p); };
    if (hipMalloc(&d_data, data.size()) != hipSuccess || hipMalloc(&d_hdr, std::max<size_t>(hdr.size() * 16, 16)) != hipSuccess ||
        hipMalloc(&d_off, uoff.size() * 8) != hipSuccess || hipMalloc(&d_side, std::max<size_t>(side.size(), 16)) != hipSuccess ||
        hipMalloc(&d_ws, std::max<uint64_t>(wsb, 256)) != hipSuccess) {
        release();
        return err(CKR_E_HIP, "[ckr] device allocation for restore failed");
    }
    int rc = CKR_OK;
    if (hipMemcpyAsync(d_data, data.data(), data.size(), hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(d_hdr, hdr.data(), hdr.size() * 16, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(d_off, uoff.data(), uoff.size() * 8, hipMemcpyHostToDevice, s) != hipSuccess ||
        (spe && hipMemcpyAsync(d_side, side.data(), side.size(), hipMemcpyHostToDevice, s) != hipSuccess))
        rc = err(CKR_E_HIP, "[ckr] upload for restore failed");
    uint64_t bad = 0;
    if (rc == CKR_OK)
        rc = ckr_decode((const uint8_t*)d_data, (const ckr_stream_header*)d_hdr, (const uint64_t*)d_off, &tab, x.n_elems,
                        x.dtype, unit, spe ? (const uint8_t*)d_side : nullptr, d_dst, d_ws, wsb, &bad, s);
    if (rc == CKR_OK && hipStreamSynchronize(s) != hipSuccess) rc = err(CKR_E_HIP, "[ckr] restore sync failed");
    release();
    if (rc == CKR_OK && bad) rc = err(CKR_E_CORRUPT, "[ckr] " + std::to_string(bad) + " lanes failed to decode in " + x.name);
    return rc;
}

}  // extern "C"
