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
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cerrno>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <filesystem>
#include <fstream>
#include <map>
#include <mutex>
#include <numeric>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "checkers_amd.h"
#include "ckr_container.h"
#include "ckr_internal.h"

namespace {

namespace fs = std::filesystem;

constexpr uint32_t kAnscMagic = 0x414E5343u;  // "ANSC"
constexpr uint32_t kMantMagic = 0x4D414E54u;  // "MANT"
constexpr uint32_t kDictMagic = 0x44494354u;  // "DICT"
constexpr uint64_t kV2Entry = 256 + 8 + 32 + 256 + 256 * 16;  // 4648
constexpr uint64_t kV4Entry = 256 + 8 + 32 + 256 + 24;        // 576
constexpr uint64_t kV4Header = 32;
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

bool unit_is_raw(const ckr_stream_header* h, uint64_t len) {
    if (h[0].byte_count != (uint32_t)len) return false;
    for (int t = 1; t < 256; t++)
        if (h[t].byte_count) return false;
    return true;
}

// ---- the writer's staging: device buffers go to the files through a pinned
// host ring.  A copy thread queues each range's D2H chunks on its own stream
// as ring slots come free; writer threads wait for a chunk's copy and pwrite
// it.  Meanwhile the calling thread encodes the next tensor into the other of
// two buffer sets.
constexpr uint64_t kSlotBytes = 32ull << 20;
constexpr uint32_t kMaxSlots = 64;

// Staging geometry: CKR_CKPT_SLOTS ring slots of 32 MiB (default 16, at most
// 64) and CKR_CKPT_WRITERS writer threads (default half the hardware threads,
// 2 to 8).  On the MI355X box (16 host cores) cfg3's 13 GB of files take
// 1.73 s with 8 slots and 8 writers, 1.08 s with 16 and 8, 0.98 s with 32 and
// 16: the writers' copies into the page cache bound it, not the 45 GB/s D2H.
uint32_t env_count(const char* name, uint32_t dflt, uint32_t lo, uint32_t hi) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    const long x = std::strtol(v, nullptr, 10);
    return (uint32_t)std::min<long>(std::max<long>(x, lo), hi);
}


struct Range {
    int fd;
    uint64_t off;
    const uint8_t* d_src;
    uint64_t len;
};

class Stager {
  public:
    Stager(uint8_t* ring, uint32_t slots, int device, hipStream_t cs, int writers)
        : ring_(ring), slots_(slots), device_(device), cs_(cs) {
        for (uint32_t i = 0; i < slots_; i++) free_.push_back(i);
        for (auto& e : slot_ev_) (void)hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventBlockingSync);
        for (auto& e : set_ev_) (void)hipEventCreateWithFlags(&e, hipEventDisableTiming);
        copier_ = std::thread([this] { copy_loop(); });
        for (int i = 0; i < writers; i++) writers_.emplace_back([this] { write_loop(); });
    }
    ~Stager() {
        finish();
        for (auto e : slot_ev_) (void)hipEventDestroy(e);
        for (auto e : set_ev_) (void)hipEventDestroy(e);
    }
    // Waits until the previous task of buffer set `set` is queued on the copy
    // stream; returns the event its copies complete at (null for a first use).
    hipEvent_t acquire_set(int set) {
        std::unique_lock<std::mutex> l(m_);
        cv_.wait(l, [&] { return !set_busy_[set]; });
        return set_used_[set] ? set_ev_[set] : nullptr;
    }
    // Copies `ranges` once `ready` (recorded on the encoding stream) has completed.
    void submit(std::vector<Range> ranges, int set, hipEvent_t ready) {
        std::lock_guard<std::mutex> l(m_);
        set_busy_[set] = set_used_[set] = true;
        tasks_.push_back({std::move(ranges), set, ready});
        cv_.notify_all();
    }
    int finish() {
        {
            std::lock_guard<std::mutex> l(m_);
            if (closed_) return rc_;
            closed_ = true;
            cv_.notify_all();
        }
        if (copier_.joinable()) copier_.join();
        {
            std::lock_guard<std::mutex> l(m_);
            writers_done_ = true;
            cv_.notify_all();
        }
        for (auto& t : writers_) t.join();
        return rc_;
    }
    int status() {
        std::lock_guard<std::mutex> l(m_);
        return rc_;
    }
    std::string message() {
        std::lock_guard<std::mutex> l(m_);
        return msg_;
    }

  private:
    struct Task {
        std::vector<Range> ranges;
        int set;
        hipEvent_t ready;
    };
    struct Chunk {
        int fd;
        uint64_t off, len;
        uint32_t slot;
    };
    void fail(int rc, const std::string& m) {  // with m_ held
        if (rc_ == CKR_OK) {
            rc_ = rc;
            msg_ = m;
        }
    }
    void copy_loop() {
        (void)hipSetDevice(device_);
        for (;;) {
            Task t;
            {
                std::unique_lock<std::mutex> l(m_);
                cv_.wait(l, [&] { return !tasks_.empty() || closed_; });
                if (tasks_.empty()) return;
                t = std::move(tasks_.front());
                tasks_.pop_front();
            }
            hipError_t e = hipStreamWaitEvent(cs_, t.ready, 0);
            for (const Range& r : t.ranges)
                for (uint64_t k = 0; k < r.len && e == hipSuccess; k += kSlotBytes) {
                    uint32_t slot;
                    {
                        std::unique_lock<std::mutex> l(m_);
                        cv_.wait(l, [&] { return !free_.empty(); });
                        if (rc_ != CKR_OK) break;
                        slot = free_.front();
                        free_.pop_front();
                    }
                    const uint64_t len = std::min(kSlotBytes, r.len - k);
                    e = hipMemcpyAsync(ring_ + slot * kSlotBytes, r.d_src + k, len, hipMemcpyDeviceToHost, cs_);
                    if (e == hipSuccess) e = hipEventRecord(slot_ev_[slot], cs_);
                    std::lock_guard<std::mutex> l(m_);
                    if (e != hipSuccess) {
                        free_.push_back(slot);
                        break;
                    }
                    chunks_.push_back({r.fd, r.off + k, len, slot});
                    cv_.notify_all();
                }
            const hipError_t e2 = hipEventRecord(set_ev_[t.set], cs_);
            std::lock_guard<std::mutex> l(m_);
            if (e != hipSuccess || e2 != hipSuccess)
                fail(CKR_E_HIP, std::string("[ckr] staging copy failed: ") + hipGetErrorString(e != hipSuccess ? e : e2));
            set_busy_[t.set] = false;
            cv_.notify_all();
        }
    }
    void write_loop() {
        (void)hipSetDevice(device_);
        for (;;) {
            Chunk c;
            {
                std::unique_lock<std::mutex> l(m_);
                cv_.wait(l, [&] { return !chunks_.empty() || writers_done_; });
                if (chunks_.empty()) return;
                c = chunks_.front();
                chunks_.pop_front();
            }
            int rc = CKR_OK;
            std::string m;
            const hipError_t e = hipEventSynchronize(slot_ev_[c.slot]);
            if (e != hipSuccess) {
                rc = CKR_E_HIP;
                m = std::string("[ckr] staging copy failed: ") + hipGetErrorString(e);
            } else if (status() == CKR_OK) {
                const uint8_t* p = ring_ + c.slot * kSlotBytes;
                for (uint64_t done = 0; done < c.len;) {
                    const ssize_t w = ::pwrite(c.fd, p + done, c.len - done, (off_t)(c.off + done));
                    if (w <= 0) {
                        if (w < 0 && errno == EINTR) continue;
                        rc = CKR_E_INVALID;
                        m = std::string("[ckr] write failed: ") + std::strerror(w < 0 ? errno : EIO);
                        break;
                    }
                    done += (uint64_t)w;
                }
            }
            std::lock_guard<std::mutex> l(m_);
            if (rc != CKR_OK) fail(rc, m);
            free_.push_back(c.slot);
            cv_.notify_all();
        }
    }

    uint8_t* ring_;
    uint32_t slots_;
    int device_;
    hipStream_t cs_;
    std::mutex m_;
    std::condition_variable cv_;
    std::deque<Task> tasks_;
    std::deque<Chunk> chunks_;
    std::deque<uint32_t> free_;
    hipEvent_t slot_ev_[kMaxSlots] = {};
    hipEvent_t set_ev_[2] = {};
    bool set_busy_[2] = {false, false}, set_used_[2] = {false, false};
    bool closed_ = false, writers_done_ = false;
    int rc_ = CKR_OK;
    std::string msg_;
    std::thread copier_;
    std::vector<std::thread> writers_;
};

// Little-endian serialisation of the small parts (headers, index entries, tables).
struct Buf {
    std::vector<uint8_t> b;
    void put(const void* p, size_t n) { b.insert(b.end(), (const uint8_t*)p, (const uint8_t*)p + n); }
    void u8(uint8_t v) { put(&v, 1); }
    void u32(uint32_t v) { put(&v, 4); }
    void u64(uint64_t v) { put(&v, 8); }
    void zeros(size_t n) { b.insert(b.end(), n, 0); }
    void name(const std::string& s) {  // 256 bytes, at most 255 copied, NUL padded
        char z[256] = {};
        std::memcpy(z, s.data(), std::min<size_t>(s.size(), 255));
        put(z, 256);
    }
};

bool pwrite_all(int fd, const void* p, uint64_t n, uint64_t off) {
    const uint8_t* q = static_cast<const uint8_t*>(p);
    while (n) {
        const ssize_t w = ::pwrite(fd, q, n, (off_t)off);
        if (w < 0 && errno == EINTR) continue;
        if (w <= 0) return false;
        q += w;
        n -= (uint64_t)w;
        off += (uint64_t)w;
    }
    return true;
}

struct Fd {
    int fd = -1;
    ~Fd() {
        if (fd >= 0) ::close(fd);
    }
};

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


// ---- the writer's buffers, kept across calls: a workspace, the histogram
// words and two sets of encode outputs that alternate between slices, plus
// the pinned host ring.  Tensors are encoded in slices of whole units under
// their whole-tensor table (units are independent streams given the table), so
// the sizes depend on the slice size and not on the largest tensor.
// ckr_ckpt_reserve sizes them ahead of a write (so that the first write
// allocates nothing), a write grows what is too small, ckr_ckpt_release frees
// everything.
struct DevBuf {
    void* p = nullptr;
    uint64_t size = 0;
};
struct WriterSet {
    DevBuf out, hdr, off, side, stored, rec, plan;
    std::vector<uint64_t> rec_off, out_off;  // host copies kept until the set is reused
};
struct WriterNeeds {
    uint64_t ws = 0, out = 0, hdr = 0, off = 0, side = 0, rec = 0, plan = 0;
};
struct WriterPool {
    std::mutex use;  // held by one writer, reserve or release for its whole duration
    int device = -1;
    DevBuf ws, hist;
    WriterSet sets[2];
    uint8_t* ring = nullptr;
    uint32_t slots = 0;
    uint64_t device_bytes() const {
        uint64_t b = ws.size + hist.size;
        for (const WriterSet& z : sets)
            for (const DevBuf* d : {&z.out, &z.hdr, &z.off, &z.side, &z.stored, &z.rec, &z.plan}) b += d->size;
        return b;
    }
};
WriterPool g_pool;

constexpr uint64_t kDefaultSliceBytes = 4ull << 30;
std::atomic<uint64_t> g_slice_bytes{0};  // 0: CKR_CKPT_SLICE_BYTES, else kDefaultSliceBytes

uint64_t slice_bytes_setting() {
    if (const uint64_t v = g_slice_bytes.load()) return v;
    if (const char* e = std::getenv("CKR_CKPT_SLICE_BYTES")) {
        const unsigned long long v = std::strtoull(e, nullptr, 10);
        if (v >= 256) return v;
    }
    return kDefaultSliceBytes;
}

// How a tensor is cut: slices of slice_units whole units (the last may hold
// fewer, and the tensor's ragged last unit); one slice when the tensor is one
// unit (v2, or a unit at least the tensor's size).
struct SliceGeom {
    uint64_t n_bytes = 0, unit = 0, nu = 0, slice_units = 0, slice_elems = 0, n_slices = 0;
    int es = 0, spe = 0;
};
SliceGeom slice_geom(uint64_t n_elems, int dtype, uint64_t unit_bytes, uint64_t slice_bytes) {
    SliceGeom g;
    g.es = ckr_element_size(dtype);
    g.spe = ckr_sidecar_bytes_per_elem(dtype);
    g.n_bytes = n_elems * (uint64_t)g.es;
    g.nu = ckr_num_units(n_elems, dtype, unit_bytes);
    if (!g.nu) return g;
    if (!unit_bytes || unit_bytes >= g.n_bytes) {
        g.unit = g.n_bytes;
        g.slice_units = g.nu;
        g.slice_elems = n_elems;
        g.n_slices = 1;
        return g;
    }
    g.unit = unit_bytes;
    g.slice_units = std::min(g.nu, std::max<uint64_t>(1, slice_bytes / unit_bytes));
    g.slice_elems = g.slice_units * unit_bytes / (uint64_t)g.es;
    g.n_slices = (g.nu + g.slice_units - 1) / g.slice_units;
    return g;
}

// Buffer sizes one tensor needs (the largest slice and the last one).
void add_needs(WriterNeeds& w, uint64_t n_elems, int dtype, uint64_t unit_bytes, uint64_t slice_bytes, bool v4) {
    const SliceGeom g = slice_geom(n_elems, dtype, unit_bytes, slice_bytes);
    if (!g.nu) return;
    const uint64_t last = n_elems - (g.n_slices - 1) * g.slice_elems;
    for (const uint64_t ne : {std::min(n_elems, g.slice_elems), last}) {
        const uint64_t nu = ckr_num_units(ne, dtype, unit_bytes);
        w.ws = std::max(w.ws, ckr_encode_workspace_bytes(ne, dtype, unit_bytes));
        w.out = std::max(w.out, ckr_encode_max_output_bytes(ne, dtype, unit_bytes));
        w.hdr = std::max(w.hdr, nu * 256 * 16);
        w.off = std::max(w.off, (nu + 1) * 8);
        w.side = std::max(w.side, ne * (uint64_t)g.spe);
        if (v4) {
            w.rec = std::max(w.rec, nu * (uint64_t)ckr::kUnitRecordMax);
            w.plan = std::max(w.plan, nu * 24);
        }
    }
}

void pool_free_all() {  // with g_pool.use held
    if (g_pool.device >= 0) {
        int cur = 0;
        (void)hipGetDevice(&cur);
        (void)hipSetDevice(g_pool.device);
        (void)hipDeviceSynchronize();
        for (DevBuf* d : {&g_pool.ws, &g_pool.hist})
            if (d->p) (void)hipFree(d->p);
        for (WriterSet& z : g_pool.sets)
            for (DevBuf* d : {&z.out, &z.hdr, &z.off, &z.side, &z.stored, &z.rec, &z.plan})
                if (d->p) (void)hipFree(d->p);
        (void)hipSetDevice(cur);
    }
    g_pool.ws = g_pool.hist = DevBuf{};
    for (WriterSet& z : g_pool.sets) z = WriterSet{};
    g_pool.device = -1;
}

// Grows the pool's buffers to `w` on the current device (with g_pool.use held).
int pool_ensure(const WriterNeeds& w, uint32_t slots) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return err(CKR_E_HIP, "[ckr] no current device");
    if (g_pool.device != dev) {
        pool_free_all();
        g_pool.device = dev;
    }
    auto grow = [](DevBuf& d, uint64_t need) {
        if (need == 0 || d.size >= need) return true;
        if (d.p) (void)hipFree(d.p);
        d = DevBuf{};
        const uint64_t b = std::max<uint64_t>(need, 256);
        if (hipMalloc(&d.p, b) != hipSuccess) {
            (void)hipGetLastError();
            d.p = nullptr;
            return false;
        }
        d.size = b;
        return true;
    };
    bool ok = grow(g_pool.ws, w.ws) && grow(g_pool.hist, 768 * 4);
    for (WriterSet& z : g_pool.sets)
        ok = ok && grow(z.out, w.out) && grow(z.hdr, w.hdr) && grow(z.off, w.off) && grow(z.side, w.side) &&
             grow(z.stored, w.rec ? w.out : 0) && grow(z.rec, w.rec) && grow(z.plan, w.plan);
    if (!ok) return err(CKR_E_HIP, "[ckr] device allocation for the checkpoint writer failed");
    if (slots && g_pool.slots < slots) {
        if (g_pool.ring) (void)hipHostFree(g_pool.ring);
        g_pool.ring = nullptr;
        g_pool.slots = 0;
        if (hipHostMalloc(reinterpret_cast<void**>(&g_pool.ring), slots * kSlotBytes, hipHostMallocDefault) != hipSuccess) {
            g_pool.ring = nullptr;
            (void)hipGetLastError();
            return err(CKR_E_HIP, "[ckr] pinned staging allocation failed");
        }
        g_pool.slots = slots;
    }
    return CKR_OK;
}

double ms_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
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
        uint64_t original = 0, n_elems = 0, data_off = 0, data_size = 0, n_units = 0, meta_off = 0, meta_size = 0;
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

int ckr_ckpt_set_slice_bytes(uint64_t bytes) {
    if (bytes && bytes < 256) return err(CKR_E_INVALID, "[ckr] slice size below 256 bytes");
    g_slice_bytes.store(bytes);
    return CKR_OK;
}

uint64_t ckr_ckpt_slice_bytes(void) { return slice_bytes_setting(); }

int ckr_ckpt_reserve(const ckr_ckpt_tensor* tensors, uint64_t n, uint64_t unit_bytes) {
    if (n && !tensors) return err(CKR_E_INVALID, "[ckr] null pointer");
    if (unit_bytes % 256) return err(CKR_E_INVALID, "[ckr] unit_bytes must be a multiple of 256");
    const uint64_t slice = slice_bytes_setting();
    WriterNeeds w;
    bool any = false;
    for (uint64_t i = 0; i < n; i++) {
        const auto& t = tensors[i];
        if (!t.d_ptr || !t.num_elements || !ckr_element_size(t.dtype)) continue;
        add_needs(w, t.num_elements, t.dtype, unit_bytes, slice, unit_bytes != 0);
        any = true;
    }
    if (!any) return CKR_OK;
    std::lock_guard<std::mutex> lk(g_pool.use);
    return pool_ensure(w, env_count("CKR_CKPT_SLOTS", 16, 2, kMaxSlots));
}

uint64_t ckr_ckpt_pool_bytes(void) {
    std::lock_guard<std::mutex> lk(g_pool.use);
    return g_pool.device_bytes();
}

void ckr_ckpt_release(void) {
    std::lock_guard<std::mutex> lk(g_pool.use);
    pool_free_all();
    if (g_pool.ring) (void)hipHostFree(g_pool.ring);
    g_pool.ring = nullptr;
    g_pool.slots = 0;
}

int ckr_ckpt_write(const char* output_dir, int rank, const ckr_ckpt_tensor* tensors, uint64_t n, uint64_t unit_bytes,
                   int repair_tables, ckr_ckpt_stats* h_stats, void* stream) {
    if (!output_dir || (n && !tensors)) return err(CKR_E_INVALID, "[ckr] null pointer");
    if (unit_bytes % 256) return err(CKR_E_INVALID, "[ckr] unit_bytes must be a multiple of 256");
    hipStream_t s = (hipStream_t)stream;
    const bool v4 = unit_bytes != 0;
    const uint64_t slice_bytes = slice_bytes_setting();
    // the tensors written, in record order, and the layout of the three files
    struct Item {
        uint64_t i;
        SliceGeom g;
        uint64_t side_off;
    };
    std::vector<Item> items;
    WriterNeeds needs;
    uint64_t side_total = 0, n_side = 0;
    for (uint64_t i = 0; i < n; i++) {
        const auto& t = tensors[i];
        if (!t.d_ptr || !t.num_elements) continue;
        const int es = ckr_element_size(t.dtype);
        if (!es) return err(CKR_E_INVALID, "[ckr] unknown dtype for tensor " + std::string(t.name ? t.name : ""));
        if (!v4 && t.num_elements * es > 0xFFFFFFFFull)
            return err(CKR_E_INVALID, "[ckr] tensor " + std::string(t.name ? t.name : "") + " needs unit_bytes (over 4 GiB)");
        Item it{i, slice_geom(t.num_elements, t.dtype, unit_bytes, slice_bytes), side_total};
        side_total += t.num_elements * (uint64_t)it.g.spe;
        n_side += it.g.spe > 0;
        add_needs(needs, t.num_elements, t.dtype, unit_bytes, slice_bytes, v4);
        items.push_back(it);
    }
    const fs::path dir(output_dir);
    std::error_code ec;
    fs::create_directories(dir / "mantissa", ec);
    fs::create_directories(dir / "tables", ec);
    if (ec) return err(CKR_E_INVALID, "[ckr] cannot create " + dir.string() + ": " + ec.message());
    const uint32_t r = (uint32_t)(rank < 0 ? 0 : rank);
    const std::string tag = "rank_" + std::to_string(r);
    const fs::path sp = dir / (tag + "_states.ansc"), mp = dir / "mantissa" / (tag + "_mantissa.mant"),
                   dp = dir / "tables" / (tag + "_tables.dict");
    Fd fs_, fm, fd_;
    fs_.fd = ::open(sp.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fs_.fd < 0) return err(CKR_E_INVALID, "[ANS] cannot open for write: " + sp.string());
    fm.fd = ::open(mp.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fm.fd < 0) return err(CKR_E_INVALID, "[ANS] cannot open mantissa for write: " + mp.string());
    fd_.fd = ::open(dp.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fd_.fd < 0) return err(CKR_E_INVALID, "[ANS] cannot open tables for write: " + dp.string());
    const uint64_t nw = items.size();
    const uint64_t data_base = v4 ? kV4Header + nw * kV4Entry : 16 + nw * kV2Entry;
    const uint64_t mant_base = 16 + n_side * kMantEntry;

    // anchors: the first record of each cluster (cluster_anchor); the table
    // owner is the first one that is compressed (compress_and_save_all :1057-1069)
    std::unordered_map<int32_t, std::string> anchor_name;
    for (uint64_t i = 0; i < n; i++)
        if (tensors[i].cluster_id >= 0 && !anchor_name.count(tensors[i].cluster_id))
            anchor_name[tensors[i].cluster_id] = tensors[i].name ? tensors[i].name : "";
    std::unordered_map<int32_t, ckr_freq_table*> cluster_table;
    std::vector<ckr_freq_table> tables(nw);

    // per written tensor: what the index needs
    struct Out {
        uint64_t data_off = 0, data_size = 0, meta_off = 0;
        bool raw = false, owns = false;
        std::string anchor;
        ckr_freq_table* table = nullptr;
        std::vector<ckr_stream_header> v2_headers;
        std::vector<uint8_t> meta;
    };
    std::vector<Out> outs(nw);

    const uint32_t slots = env_count("CKR_CKPT_SLOTS", 16, 2, kMaxSlots);
    std::unique_lock<std::mutex> pool_lock(g_pool.use);
    if (nw) {
        if (int rc = pool_ensure(needs, slots)) return rc;
    }
    hipStream_t cs = nullptr;
    hipEvent_t ready[2] = {nullptr, nullptr};
    auto release = [&]() {
        for (auto e : ready)
            if (e) (void)hipEventDestroy(e);
        if (cs) (void)hipStreamDestroy(cs);
    };
    if (nw && (hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess ||
               hipEventCreateWithFlags(&ready[0], hipEventDisableTiming) != hipSuccess ||
               hipEventCreateWithFlags(&ready[1], hipEventDisableTiming) != hipSuccess)) {
        (void)hipGetLastError();
        release();
        return err(CKR_E_HIP, "[ckr] stream or event creation for the checkpoint writer failed");
    }
    int device = 0;
    if (nw) (void)hipGetDevice(&device);
    const unsigned hw = std::max(2u, std::thread::hardware_concurrency());
    int rc = CKR_OK;
    uint64_t data_cursor = 0, meta_cursor = 0;
    if (nw) {
        Stager st(g_pool.ring, slots, device, cs, (int)env_count("CKR_CKPT_WRITERS", std::min(8u, std::max(2u, hw / 2)), 1, 32));
        uint32_t* d_hist = static_cast<uint32_t*>(g_pool.hist.p);
        uint64_t j = 0;  // slices so far: slice j is encoded into buffer set j & 1
        for (uint64_t k = 0; k < nw && rc == CKR_OK; k++) {
            const Item& it = items[k];
            const SliceGeom& g = it.g;
            const auto& t = tensors[it.i];
            Out& o = outs[k];
            const bool singleton = t.cluster_id < 0;
            auto cit = cluster_table.find(t.cluster_id);
            o.owns = singleton || cit == cluster_table.end();
            ckr_freq_table* tab = &tables[k];
            uint32_t tsum = CKR_M;
            double hist_ms = 0, table_ms = 0, encode_ms = 0, copy_ms = 0;
            // the table: owners count the whole tensor (masked histogram and the
            // two live planes' histograms, which size the encoder's slots); members
            // take their cluster's
            uint32_t planes[768];
            const uint32_t* h_planes = nullptr;
            if (o.owns) {
                auto t0 = std::chrono::steady_clock::now();
                rc = ckr_byte_histogram_planes(t.d_ptr, t.num_elements, t.dtype, d_hist, s);
                if (rc != CKR_OK) break;
                if (hipMemcpyAsync(planes, d_hist, sizeof(planes), hipMemcpyDeviceToHost, s) != hipSuccess ||
                    hipStreamSynchronize(s) != hipSuccess) {
                    rc = err(CKR_E_HIP, "[ckr] histogram read-back failed");
                    break;
                }
                hist_ms = ms_since(t0);
                t0 = std::chrono::steady_clock::now();
                rc = ckr_build_table(planes, singleton ? 0 : 1, tab, &tsum);
                if (rc != CKR_OK) break;
                if (repair_tables && tsum > CKR_M) repair_table(tab);
                table_ms = ms_since(t0);
                if (g.spe) h_planes = planes + 256;
                if (!singleton) cluster_table[t.cluster_id] = tab;
                o.table = tab;
            } else {
                tab = cit->second;
                tsum = tab->cum_freq[256];
                o.anchor = anchor_name[t.cluster_id];
            }
            o.raw = true;
            o.data_off = data_cursor;
            o.meta_off = meta_cursor;
            uint64_t total = 0, stored_total = 0;
            for (uint64_t sl = 0; sl < g.n_slices && rc == CKR_OK; sl++, j++) {
                WriterSet& z = g_pool.sets[j & 1];
                if (hipEvent_t prev = st.acquire_set((int)(j & 1))) {
                    if (hipStreamWaitEvent(s, prev, 0) != hipSuccess) { rc = err(CKR_E_HIP, "[ckr] stream wait failed"); break; }
                }
                if ((rc = st.status()) != CKR_OK) break;
                const uint64_t e0 = sl * g.slice_elems;
                const uint64_t ne = std::min(g.slice_elems, t.num_elements - e0);
                const uint64_t nb = ne * (uint64_t)g.es;
                const uint64_t snu = ckr_num_units(ne, t.dtype, unit_bytes);
                const uint8_t* src = static_cast<const uint8_t*>(t.d_ptr) + e0 * (uint64_t)g.es;
                auto t0 = std::chrono::steady_clock::now();
                uint64_t stotal = 0;
                rc = ckr::encode_slice_of_counted(src, ne, t.dtype, tab, h_planes, unit_bytes, (uint8_t*)z.out.p, z.out.size,
                                       (ckr_stream_header*)z.hdr.p, (uint64_t*)z.off.p, (uint8_t*)z.side.p, g_pool.ws.p,
                                       g_pool.ws.size, &stotal, s);
                encode_ms += ms_since(t0);
                if (rc != CKR_OK) break;
                total += stotal;
                t0 = std::chrono::steady_clock::now();
                const void* stored = z.out.p;
                uint64_t stored_size = stotal;
                if (v4) {
                    // unit records and the bytes a unit keeps: sizes, host scan, pack
                    const ckr::UnitGeomArg ug{nb, std::min(g.unit, nb), snu, g.es, g.spe};
                    const ckr::ZeroLanes zl = ckr::zero_lanes(tab, nb, ug.unit);
                    uint32_t* d_rs = static_cast<uint32_t*>(z.plan.p);
                    uint32_t* d_ds = d_rs + snu;
                    uint64_t* d_ro = reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(z.plan.p) + snu * 8);
                    uint64_t* d_oo = d_ro + snu;
                    std::vector<uint32_t> sz(2 * snu);
                    hipError_t e = ckr::launch_unit_plan((const ckr_stream_header*)z.hdr.p, ug, zl.arg, d_rs, d_ds, s);
                    if (e == hipSuccess) e = hipMemcpyAsync(sz.data(), d_rs, sz.size() * 4, hipMemcpyDeviceToHost, s);
                    if (e == hipSuccess) e = hipStreamSynchronize(s);
                    if (e != hipSuccess) { rc = err(CKR_E_HIP, std::string("[ckr] unit plan failed: ") + hipGetErrorString(e)); break; }
                    z.rec_off.assign(snu, 0);
                    z.out_off.assign(snu, 0);
                    uint64_t ra = 0, oa = 0;
                    for (uint64_t u = 0; u < snu; u++) {
                        z.rec_off[u] = ra;
                        z.out_off[u] = oa;
                        ra += sz[u];
                        oa += sz[snu + u];
                    }
                    e = hipMemcpyAsync(d_ro, z.rec_off.data(), snu * 8, hipMemcpyHostToDevice, s);
                    if (e == hipSuccess) e = hipMemcpyAsync(d_oo, z.out_off.data(), snu * 8, hipMemcpyHostToDevice, s);
                    if (e == hipSuccess)
                        e = ckr::launch_unit_pack((const uint8_t*)z.out.p, (const uint64_t*)z.off.p,
                                                  (const ckr_stream_header*)z.hdr.p, ug, zl.arg, d_ro, d_oo,
                                                  (uint8_t*)z.rec.p, (uint8_t*)z.stored.p, s);
                    const uint64_t m0 = o.meta.size();
                    o.meta.resize(m0 + ra);
                    if (e == hipSuccess && ra) e = hipMemcpyAsync(o.meta.data() + m0, z.rec.p, ra, hipMemcpyDeviceToHost, s);
                    if (e == hipSuccess) e = hipStreamSynchronize(s);
                    if (e != hipSuccess) { rc = err(CKR_E_HIP, std::string("[ckr] unit pack failed: ") + hipGetErrorString(e)); break; }
                    for (uint64_t u = 0, p = m0; u < snu && o.raw; u++) {
                        o.raw = o.meta[p] == 1;
                        p += sz[u];
                    }
                    stored = z.stored.p;
                    stored_size = oa;
                } else {
                    o.v2_headers.resize(256);
                    if (hipMemcpyAsync(o.v2_headers.data(), z.hdr.p, 256 * 16, hipMemcpyDeviceToHost, s) != hipSuccess ||
                        hipStreamSynchronize(s) != hipSuccess) {
                        rc = err(CKR_E_HIP, "[ckr] copy of stream headers failed");
                        break;
                    }
                    o.raw = unit_is_raw(o.v2_headers.data(), nb);
                }
                copy_ms += ms_since(t0);
                if (hipEventRecord(ready[j & 1], s) != hipSuccess) { rc = err(CKR_E_HIP, "[ckr] event record failed"); break; }
                std::vector<Range> ranges;
                if (stored_size)
                    ranges.push_back({fs_.fd, data_base + o.data_off + stored_total, (const uint8_t*)stored, stored_size});
                if (g.spe)
                    ranges.push_back({fm.fd, mant_base + it.side_off + e0 * (uint64_t)g.spe, (const uint8_t*)z.side.p,
                                      ne * (uint64_t)g.spe});
                st.submit(std::move(ranges), (int)(j & 1), ready[j & 1]);
                stored_total += stored_size;
            }
            if (rc != CKR_OK) break;
            o.data_size = stored_total;
            data_cursor += stored_total;
            meta_cursor += o.meta.size();
            if (h_stats) {
                ckr_ckpt_stats& hs = h_stats[k];
                std::memset(&hs, 0, sizeof(hs));
                hs.record_index = it.i;
                hs.original_bytes = g.n_bytes;
                hs.ans_bytes = total;
                hs.sidecar_bytes = t.num_elements * (uint64_t)g.spe;
                hs.owns_table = o.owns;
                hs.table_sum = tsum;
                hs.table_repaired = (o.owns && repair_tables && tsum > CKR_M) ? 1 : 0;
                hs.n_slices = (uint32_t)g.n_slices;
                hs.stored_bytes = stored_total;
                hs.record_bytes = o.meta.size();
                hs.hist_ms = hist_ms;
                hs.table_ms = table_ms;
                hs.encode_ms = encode_ms;
                hs.copy_ms = copy_ms;
            }
        }
        const int src = st.finish();
        if (rc == CKR_OK && src != CKR_OK) rc = err(src, st.message());
    }
    release();
    pool_lock.unlock();
    if (rc != CKR_OK) return rc;

    // the small parts: states header, index and (v4) unit records; mantissa
    // index; tables
    Buf b;
    b.u32(kAnscMagic);
    b.u32(v4 ? 4u : 2u);
    b.u32(r);
    b.u32((uint32_t)nw);
    if (v4) {
        b.u64(unit_bytes);
        b.u64(data_base + data_cursor);  // where the unit records begin
    }
    for (uint64_t k = 0; k < nw; k++) {
        const auto& t = tensors[items[k].i];
        const Out& o = outs[k];
        b.name(t.name ? t.name : "");
        b.u8((uint8_t)t.dtype);
        b.u8(o.raw ? 1 : 0);
        b.u8(o.owns ? 1 : 0);
        b.zeros(5);
        b.u64(items[k].g.n_bytes);
        b.u64(t.num_elements);
        b.u64(o.data_off);
        b.u64(o.data_size);
        b.name(o.owns ? std::string() : o.anchor);
        if (v4) {
            b.u64(items[k].g.nu);
            b.u64(o.meta_off);
            b.u64(o.meta.size());
        } else {
            b.put(o.v2_headers.data(), 256 * 16);
        }
    }
    bool wok = pwrite_all(fs_.fd, b.b.data(), b.b.size(), 0);
    for (uint64_t k = 0; k < nw && v4 && wok; k++)
        wok = pwrite_all(fs_.fd, outs[k].meta.data(), outs[k].meta.size(), data_base + data_cursor + outs[k].meta_off);
    Buf m;
    m.u32(kMantMagic);
    m.u32(2u);
    m.u32(r);
    m.u32((uint32_t)n_side);
    for (uint64_t k = 0; k < nw; k++) {
        if (!items[k].g.spe) continue;
        const auto& t = tensors[items[k].i];
        m.name(t.name ? t.name : "");
        m.u8((uint8_t)t.dtype);
        m.u8((uint8_t)items[k].g.spe);
        m.zeros(6);
        m.u64(t.num_elements);
        m.u64(items[k].side_off);
        m.u64(t.num_elements * (uint64_t)items[k].g.spe);
    }
    wok = wok && pwrite_all(fm.fd, m.b.data(), m.b.size(), 0);
    Buf d;
    uint32_t owners = 0;
    for (const Out& o : outs) owners += o.owns;
    d.u32(kDictMagic);
    d.u32(1u);
    d.u32(r);
    d.u32(owners);
    for (uint64_t k = 0; k < nw; k++) {
        if (!outs[k].owns) continue;
        d.name(tensors[items[k].i].name ? tensors[items[k].i].name : "");
        d.put(outs[k].table->norm_freq, 256 * 4);
        d.put(outs[k].table->cum_freq, 257 * 4);
    }
    wok = wok && pwrite_all(fd_.fd, d.b.data(), d.b.size(), 0);
    if (!wok) return err(CKR_E_INVALID, std::string("[ckr] write failed in ") + dir.string() + ": " + std::strerror(errno));
    return CKR_OK;
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
    if (!read_at(f, 0, h, 16) || h[0] != kAnscMagic || (h[1] != 2 && h[1] != 4))
        return err(CKR_E_CORRUPT, "[ckr] not an .ansc v2/v4 file: " + sp.string());
    c->version = h[1];
    c->rank = h[2];
    const uint32_t nt = h[3];
    uint64_t pos = 16;
    if (c->version == 4) {
        uint64_t u[2];
        if (!read_at(f, 16, u, 16)) return err(CKR_E_CORRUPT, "[ckr] truncated header");
        c->unit_bytes = u[0];
        c->meta_base = u[1];
        pos = kV4Header;
        if (c->unit_bytes == 0 || c->unit_bytes % 256) return err(CKR_E_CORRUPT, "[ckr] bad unit size in " + sp.string());
    }
    const uint64_t esz = c->version == 4 ? kV4Entry : kV2Entry;
    std::vector<uint8_t> buf(esz);
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
        if (c->version == 4) {
            std::memcpy(&e.n_units, b + 552, 8);
            std::memcpy(&e.meta_off, b + 560, 8);
            std::memcpy(&e.meta_size, b + 568, 8);
        } else {
            e.n_units = 1;
            e.v2_headers.resize(256);
            std::memcpy(e.v2_headers.data(), b + 552, 256 * 16);
        }
        c->entries.push_back(std::move(e));
    }
    c->data_base = pos;
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
    e->unit_bytes = c->version == 4 ? c->unit_bytes : 0;
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
    const uint64_t unit = c->version == 4 ? c->unit_bytes : 0;
    const uint64_t nu = ckr_num_units(x.n_elems, x.dtype, unit);
    if (nu != x.n_units) return err(CKR_E_CORRUPT, "[ckr] unit count mismatch for " + x.name);
    const fs::path sp = c->dir / ("rank_" + std::to_string(c->rank) + "_states.ansc");
    std::error_code fec;
    const uint64_t fsize = fs::file_size(sp, fec);
    // every unit has a record of at least one byte (v4); sizes within the file
    if (fec || x.data_size > fsize || x.meta_size > fsize || (c->version == 4 && nu > x.meta_size))
        return err(CKR_E_CORRUPT, "[ckr] entry " + x.name + " does not fit its file");
    std::ifstream f(sp, std::ios::binary);
    std::vector<ckr_stream_header> hdr;
    std::vector<uint64_t> uoff;
    std::vector<uint8_t> data(std::max<uint64_t>(x.data_size, 1));
    if (x.data_size && !read_at(f, c->data_base + x.data_off, data.data(), x.data_size))
        return err(CKR_E_CORRUPT, "[ckr] truncated data for " + x.name);
    const uint64_t ulen = unit ? std::min(unit, x.original) : x.original;
    if (c->version == 4) {
        std::vector<uint8_t> meta(std::max<uint64_t>(x.meta_size, 1));
        if (!read_at(f, c->meta_base + x.meta_off, meta.data(), x.meta_size))
            return err(CKR_E_CORRUPT, "[ckr] truncated unit records for " + x.name);
        const ckr::ZeroLanes zl = ckr::zero_lanes(&tab, x.original, ulen);
        std::vector<uint8_t> full;
        std::string why;
        if (ckr::expand_units(meta.data(), x.meta_size, data.data(), x.data_size, x.original, ulen, es, (int)spe, zl,
                              hdr, uoff, full, why) != CKR_OK)
            return err(CKR_E_CORRUPT, "[ckr] corrupt unit records for " + x.name + ": " + why);
        data.swap(full);
        if (data.empty()) data.resize(1);
    } else {
        hdr = x.v2_headers;
        uoff = {0, x.data_size};
    }
    const uint64_t full_size = uoff.empty() ? 0 : uoff.back();
    if (int rc = check_unit_metadata(hdr, uoff, nu, x.original, ulen, full_size, x.name)) return rc;
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
