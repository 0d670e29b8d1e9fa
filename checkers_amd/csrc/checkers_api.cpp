// checkers_amd/csrc/checkers_api.cpp — checkers::initialize_context /
// analyze_tensors / compress_and_save (include/checkers_api.hpp) over the C ABI.
//
// Reference (paths relative to the reference tree):
//   initialize_context, tensor discovery     src/api.cpp:27-887, :899-1031
//   analyze_tensors                          src/api.cpp:1033-1253
//   compress_and_save                        src/api.cpp:1255-1299
//   MemoryManager::process_batch             src/MemoryManager.cpp:306-690
// Discovery follows api.cpp: the ZeRO-3 flat-group walk when the optimizer has
// fp16/fp32_partitioned_groups_flat, else one record per named parameter from
// its ds_tensor partition, the parameter, .data or _hp_mapping.hp_tensor.
// Record names, order and dtype tags are the reference's, including
// parse_dtype's order of tests, which tags bfloat16 tensors as float16.
// Records are submitted in discovery order on the calling thread (the
// reference's background_threads == 1 ordering; the argument is accepted and
// checked).  Where the reference would hand a kernel a pointer it cannot use,
// the tensor is skipped and counted instead: tensors that are not on a GPU.
//
// The module has no link-time dependency on libcheckers_amd.so or the HIP
// runtime: on first use it imports torch (when importable), so that torch's
// bundled HIP runtime is loaded first, then dlopens libcheckers_amd.so, whose
// libamdhip64.so.7 then resolves to that runtime.  Linking them directly would
// load /opt/rocm's runtime as well when the module is imported before torch,
// and two HIP runtimes in one process do not share devices.
#include "checkers_api.hpp"

#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "checkers_amd.h"

namespace checkers {

namespace {

constexpr uint64_t kSlabAlign = 256;  // MemoryManager::alignment_bytes_ (MemoryManager.hpp:235)

// libcheckers_amd.so: CHECKERS_AMD_LIB, else checkers_amd/ beside this module.
void* library() {
    static void* handle = [] {
        try {
            py::module_::import("torch");
        } catch (py::error_already_set&) {
            // no torch: the library loads whichever runtime the loader finds
        }
        std::string path;
        if (const char* e = std::getenv("CHECKERS_AMD_LIB")) {
            path = e;
        } else {
            Dl_info info{};
            if (!dladdr(reinterpret_cast<void*>(&library), &info) || !info.dli_fname)
                throw std::runtime_error("cannot locate the checkers_py module");
            path = info.dli_fname;
            path = path.substr(0, path.find_last_of('/') + 1) + "checkers_amd/libcheckers_amd.so";
        }
        void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
        if (!h) throw std::runtime_error("cannot load " + path + ": " + dlerror());
        return h;
    }();
    return handle;
}

// A symbol of the library or of the HIP runtime it links.
template <typename F>
F bound(const char* name) {
    void* p = dlsym(library(), name);
    if (!p) throw std::runtime_error(std::string("missing symbol ") + name);
    return reinterpret_cast<F>(p);
}
#define CKR(f) bound<decltype(&f)>(#f)
#define HIPFN(f, ...) bound<hipError_t (*)(__VA_ARGS__)>(#f)
const char* hip_error(hipError_t e) { return bound<const char* (*)(hipError_t)>("hipGetErrorString")(e); }

// A discovered tensor: its record (pointer, stats buffers, sizes, tags), the
// Python object that keeps its memory alive, and its layout.
struct Record {
    std::string name;
    py::object holder;
    ckr_device_tensor_record rec{};
    int elem_size = 0;
    std::vector<int64_t> shape, strides;
};

struct Context {
    int rank = -1;
    size_t bins = 256;
    size_t threads = 1;
    size_t skipped = 0;
    std::vector<Record> recs;
    ckr_arena* arena = nullptr;
    void* analyze_ws = nullptr;  // the statistics pass's workspace, kept for the context's life
    uint64_t analyze_wsb = 0;
    std::vector<int32_t> cluster_of;  // after analyze_tensors
    ~Context() {
        if (analyze_ws) (void)HIPFN(hipFree, void*)(analyze_ws);
        if (arena) CKR(ckr_arena_destroy)(arena);
        CKR(ckr_ckpt_release)();  // the checkpoint writer's buffers, reserved for this context
    }
};

// The context holds Python objects and device memory, so it must go while the
// interpreter and the HIP runtime are still up: a hook registered with Python's
// atexit releases it.  A static destructor would run after the interpreter
// has finalised.
Context* g_ctx = nullptr;

void release_context() {
    delete g_ctx;
    g_ctx = nullptr;
}

void register_release_at_exit() {
    static bool done = false;
    if (done) return;
    py::module_::import("atexit").attr("register")(py::cpp_function(&release_context));
    done = true;
}

void check(int rc, const char* what) {
    if (rc != CKR_OK) throw std::runtime_error(std::string(what) + ": " + CKR(ckr_last_error)());
}

// torch's current stream on the current device when torch is loaded (the
// tensors' producers queue there), else the null stream.
void* current_stream() {
    try {
        py::object torch = py::module_::import("torch");
        return reinterpret_cast<void*>(torch.attr("cuda").attr("current_stream")().attr("cuda_stream").cast<uintptr_t>());
    } catch (...) {
        PyErr_Clear();
        return nullptr;
    }
}

// CHECKERS_UNIT_BYTES: unit size of the chunked states file (.ansc v4,
// default 65536); 0 writes the reference's v2 layout (one stream per tensor,
// tensors below 4 GiB, encoded 256 lanes wide only).
uint64_t unit_bytes_setting() {
    uint64_t unit = 65536;
    if (const char* v = std::getenv("CHECKERS_UNIT_BYTES")) unit = std::strtoull(v, nullptr, 10);
    return unit;
}

// parse_dtype (api.cpp:887-893): substring tests in this order.
uint8_t parse_dtype(const std::string& s) {
    if (s.find("float32") != std::string::npos) return CKR_F32;
    if (s.find("float16") != std::string::npos) return CKR_F16;
    if (s.find("bfloat16") != std::string::npos) return CKR_BF16;
    if (s.find("int8") != std::string::npos) return CKR_I8;
    return CKR_UNKNOWN;
}

// extract_rank (api.cpp:27-35).
int extract_rank(py::object engine, const char* attr, const char* env) {
    if (py::hasattr(engine, attr)) return engine.attr(attr).cast<int>();
    if (const char* v = std::getenv(env)) return std::atoi(v);
    return -1;
}

// resolve_optimizer (api.cpp:67-78).
py::object resolve_optimizer(py::object engine, py::object optimizer) {
    if (!optimizer.is_none()) return optimizer;
    if (py::hasattr(engine, "optimizer")) {
        py::object o = engine.attr("optimizer");
        if (!o.is_none()) return o;
    }
    return py::none();
}

// extract_group_rank (api.cpp:690-710): rank inside the parameter's process group.
int extract_group_rank(py::object param, int fallback) {
    if (!py::hasattr(param, "ds_process_group")) return fallback;
    try {
        py::object dist = py::module_::import("torch.distributed");
        if (py::hasattr(dist, "is_initialized") && !dist.attr("is_initialized")().cast<bool>()) return fallback;
        py::object group = param.attr("ds_process_group");
        if (group.is_none()) return fallback;
        return dist.attr("get_rank")(py::arg("group") = group).cast<int>();
    } catch (...) {
        PyErr_Clear();
        return fallback;
    }
}

// A tensor-like handle's pointer, size and layout (try_tensor_like, api.cpp:790-851).
// resident: when nonzero, only the first `resident` elements (a 1-D partition).
bool tensor_record(py::handle h, const std::string& name, size_t resident, Record* out) {
    if (!py::hasattr(h, "data_ptr")) return false;
    const uintptr_t ptr = h.attr("data_ptr")().cast<uintptr_t>();
    if (!ptr) return false;
    if (py::hasattr(h, "is_cuda") && !h.attr("is_cuda").cast<bool>()) return false;  // host tensor
    const size_t es = py::hasattr(h, "element_size") ? h.attr("element_size")().cast<size_t>() : 0;
    size_t numel = py::hasattr(h, "numel") ? h.attr("numel")().cast<size_t>() : 0;
    if (!es || !numel) return false;
    std::string dt = "unknown";
    if (py::hasattr(h, "dtype")) dt = py::str(h.attr("dtype")).cast<std::string>();
    Record r;
    r.name = name;
    r.holder = py::reinterpret_borrow<py::object>(h);
    r.elem_size = (int)es;
    r.rec.d_ptr = reinterpret_cast<void*>(ptr);
    r.rec.data_type = parse_dtype(dt);
    if (resident) {
        numel = std::min(numel, resident);
        r.shape = {(int64_t)numel};
        r.strides = {1};
    } else {
        if (py::hasattr(h, "shape"))
            for (auto d : py::list(h.attr("shape"))) r.shape.push_back(d.cast<int64_t>());
        if (py::hasattr(h, "stride"))
            for (auto d : py::list(h.attr("stride")())) r.strides.push_back(d.cast<int64_t>());
    }
    r.rec.num_elements = numel;
    *out = std::move(r);
    return true;
}

// try_zero_partitioned_tensor (api.cpp:712-787): this rank's resident part of ds_tensor.
bool zero_partition(py::object param, py::handle h, int fallback_rank, const std::string& name, Record* out) {
    size_t logical = 0, part = 0;
    if (py::hasattr(param, "ds_numel")) logical = param.attr("ds_numel").cast<size_t>();
    else if (py::hasattr(h, "numel")) logical = h.attr("numel")().cast<size_t>();
    if (py::hasattr(param, "partition_numel")) part = param.attr("partition_numel")().cast<size_t>();
    else if (py::hasattr(h, "ds_numel")) part = h.attr("ds_numel").cast<size_t>();
    if (!logical || !part) return false;
    const int r = extract_group_rank(param, fallback_rank);
    const size_t off = r < 0 ? 0 : (size_t)r * part;
    if (off >= logical) return false;
    const size_t resident = std::min(part, logical - off);
    return resident && tensor_record(h, name, resident, out);
}

// extract_tensor (api.cpp:852-885).
bool extract_tensor(py::object param, int rank, const std::string& name, Record* out) {
    if (py::hasattr(param, "ds_tensor") && !param.attr("ds_tensor").is_none()) {
        py::object ds = param.attr("ds_tensor");
        if (zero_partition(param, ds, rank, name, out)) return true;
        if (tensor_record(ds, name, 0, out)) return true;
    }
    if (tensor_record(param, name, 0, out)) return true;
    if (py::hasattr(param, "data") && tensor_record(param.attr("data"), name, 0, out)) return true;
    if (py::hasattr(param, "_hp_mapping") && !param.attr("_hp_mapping").is_none()) {
        py::object hp = param.attr("_hp_mapping");
        if (py::hasattr(hp, "hp_tensor") && !hp.attr("hp_tensor").is_none() &&
            tensor_record(hp.attr("hp_tensor"), name, 0, out))
            return true;
    }
    return false;
}

// submit_partition_slice (api.cpp:206-241): flat.narrow(0, offset, numel).
bool partition_slice(py::object flat, size_t offset, size_t numel, const std::string& name, Record* out) {
    if (!numel) return false;
    py::object slice = flat.attr("narrow")(0, offset, numel);
    return tensor_record(slice, name, numel, out);
}

// discover_zero3_flat_states (api.cpp:416-685).
void discover_zero3(Context& c, py::object opt, const py::list& named) {
    py::list fp32, fp16;
    if (py::hasattr(opt, "fp32_partitioned_groups_flat")) fp32 = py::list(opt.attr("fp32_partitioned_groups_flat"));
    if (py::hasattr(opt, "fp16_partitioned_groups_flat")) fp16 = py::list(opt.attr("fp16_partitioned_groups_flat"));
    py::dict state;
    bool has_state = false;
    if (py::hasattr(opt, "optimizer")) {
        py::object base = opt.attr("optimizer");
        if (!base.is_none() && py::hasattr(base, "state")) {
            py::object raw = base.attr("state");
            if (!raw.is_none() && py::isinstance<py::dict>(raw)) {
                state = raw.cast<py::dict>();
                has_state = !state.empty();
            }
        }
    }
    const bool has_pos = py::hasattr(opt, "grad_position") && py::hasattr(opt, "get_param_id");
    const size_t ng = fp32.size();
    if (!ng) return;
    struct P {
        std::string name;
        py::object param;
        size_t foff, fnumel, dsn;
    };
    std::vector<std::vector<P>> groups(ng);
    if (has_pos) {
        for (auto item : named) {
            py::tuple t = item.cast<py::tuple>();
            const std::string pname = t[0].cast<std::string>();
            py::object p = t[1];
            if (!py::hasattr(p, "requires_grad") || !p.attr("requires_grad").cast<bool>() || !py::hasattr(p, "ds_numel"))
                continue;
            try {
                py::object pid = opt.attr("get_param_id")(p);
                py::object loc = opt.attr("grad_position").attr("get")(pid, py::none());
                if (loc.is_none()) continue;
                py::list l(loc);
                const size_t g = l[0].cast<size_t>(), foff = l[1].cast<size_t>(), fn = l[2].cast<size_t>();
                const size_t dsn = p.attr("ds_numel").cast<size_t>();
                if (g < ng && fn > 0 && dsn > 0) groups[g].push_back({pname, p, foff, fn, dsn});
            } catch (...) {
                PyErr_Clear();
            }
        }
        for (auto& gp : groups)
            std::sort(gp.begin(), gp.end(), [](const P& a, const P& b) { return a.foff < b.foff; });
    }
    for (size_t g = 0; g < ng; g++) {
        if (groups[g].empty()) continue;
        py::object f32 = fp32[g];
        const size_t size = f32.attr("numel")().cast<size_t>();
        if (!size) continue;
        size_t total = 0;
        for (const auto& p : groups[g]) total += p.dsn;
        const size_t lo = (size_t)std::max(c.rank, 0) * size;
        const size_t hi = std::min(((size_t)std::max(c.rank, 0) + 1) * size, total);
        py::object f16 = g < fp16.size() ? py::object(fp16[g]) : py::none();
        py::object ea = py::none(), easq = py::none();
        if (has_state && state.contains(f32)) {
            py::dict st = state[f32].cast<py::dict>();
            if (st.contains("exp_avg")) ea = st["exp_avg"];
            if (st.contains("exp_avg_sq")) easq = st["exp_avg_sq"];
        }
        size_t pos = 0;
        for (const auto& p : groups[g]) {
            const size_t s = pos, e = pos + p.dsn;
            pos = e;
            if (e <= lo || s >= hi) {
                c.skipped++;
                continue;
            }
            size_t got = 0;
            Record r;
            if (!f16.is_none()) {
                if (partition_slice(f16, p.foff, p.fnumel, p.name, &r)) { c.recs.push_back(std::move(r)); got++; }
            } else if (py::hasattr(p.param, "ds_tensor") && !p.param.attr("ds_tensor").is_none()) {
                if (zero_partition(p.param, p.param.attr("ds_tensor"), c.rank, p.name, &r)) {
                    c.recs.push_back(std::move(r));
                    got++;
                }
            }
            if (partition_slice(f32, p.foff, p.fnumel, "master_weights::" + p.name, &r)) { c.recs.push_back(std::move(r)); got++; }
            if (has_state && !ea.is_none() &&
                partition_slice(ea, p.foff, p.fnumel, "optimizer.exp_avg::" + p.name, &r)) {
                c.recs.push_back(std::move(r));
                got++;
            }
            if (has_state && !easq.is_none() &&
                partition_slice(easq, p.foff, p.fnumel, "optimizer.exp_avg_sq::" + p.name, &r)) {
                c.recs.push_back(std::move(r));
                got++;
            }
            if (!got) c.skipped++;
        }
    }
}

// check_and_fix_contiguity (MemoryManager.cpp:709-740): 0-dim ⇒ scalar, row-major
// strides ⇒ contiguous, else non-contiguous (gathered).
uint8_t contiguity(const Record& r) {
    if (r.shape.empty()) return 2;
    if (r.strides.empty()) return 0;
    int64_t expected = 1;
    for (int d = (int)r.shape.size() - 1; d >= 0; d--) {
        if (r.shape[d] != 1 && r.strides[d] != expected) return 1;
        expected *= r.shape[d];
    }
    return 0;
}

// Arena for the context: every record's statistics slab, then the contiguous
// copies of the non-contiguous tensors (make_contiguous, TensorResource.cpp:85-153).
void place_records(Context& c, void* stream) {
    uint64_t cap = 0;
    const uint64_t slab = CKR(ckr_stats_slab_bytes)((uint32_t)c.bins, kSlabAlign);
    std::vector<uint8_t> contig(c.recs.size());
    for (size_t i = 0; i < c.recs.size(); i++) {
        contig[i] = contiguity(c.recs[i]);
        cap += slab;
        if (contig[i] == 1) cap += (c.recs[i].rec.num_elements * c.recs[i].elem_size + kSlabAlign - 1) / kSlabAlign * kSlabAlign;
    }
    check(CKR(ckr_arena_create)(cap, &c.arena), "arena");
    void* slabs = nullptr;
    if (!c.recs.empty()) {
        check(CKR(ckr_arena_alloc)(c.arena, slab * c.recs.size(), kSlabAlign, &slabs), "arena");
        const hipError_t e = HIPFN(hipMemsetAsync, void*, int, size_t, hipStream_t)(slabs, 0, slab * c.recs.size(), (hipStream_t)stream);
        if (e != hipSuccess) throw std::runtime_error(std::string("slab clear: ") + hip_error(e));
    }
    for (size_t i = 0; i < c.recs.size(); i++) {
        Record& r = c.recs[i];
        check(CKR(ckr_carve_stats_slab)(static_cast<uint8_t*>(slabs) + i * slab, (uint32_t)c.bins, kSlabAlign, &r.rec),
              "slab carving");
        r.rec.name = r.name.c_str();
        if (contig[i] == 1) {
            void* dst = nullptr;
            check(CKR(ckr_arena_alloc)(c.arena, r.rec.num_elements * r.elem_size, kSlabAlign, &dst), "arena");
            check(CKR(ckr_make_contiguous)(r.rec.d_ptr, (int)r.shape.size(), r.shape.data(), r.strides.data(), r.elem_size,
                                      dst, stream),
                  "make_contiguous");
            r.rec.d_ptr = dst;
            contig[i] = 0;
        }
        r.rec.contiguity = contig[i];
    }
}

// CHECKERS_LOG: where compress_and_save reports what the reference's logger
// records per tensor and in total (src/ANSCompressor.cpp:1292-1312,
// :1387-1399, same fields and prefix): unset or empty, nowhere; "stderr" or
// "1", standard error; anything else, a file the lines are appended to.
void log_compress_stats(const Context& c, const std::vector<ckr_ckpt_tensor>& ts,
                        const std::vector<ckr_ckpt_stats>& stats, double wall_ms, const std::string& dir,
                        uint64_t unit) {
    const char* where = std::getenv("CHECKERS_LOG");
    if (!where || !*where) return;
    std::ostringstream o;
    const std::string lp = "[ANS][rank=" + std::to_string(c.rank) + "]";
    size_t written = 0;
    double compute_ms = 0;
    for (const ckr_ckpt_tensor& t : ts) written += (t.d_ptr && t.num_elements) ? 1 : 0;
    for (size_t k = 0; k < written; k++) {
        const ckr_ckpt_stats& s = stats[k];
        const double ans_ratio = s.ans_bytes ? (double)s.original_bytes / (double)s.ans_bytes : 1.0;
        const double disk_ratio =
            s.original_bytes ? (double)s.original_bytes / (double)(s.ans_bytes + s.sidecar_bytes) : 1.0;
        compute_ms += s.hist_ms + s.table_ms + s.encode_ms + s.copy_ms;
        o << lp << "[tensor] name=" << ts[s.record_index].name << " original_bytes=" << s.original_bytes
          << " ans_bytes=" << s.ans_bytes << " sidecar_bytes=" << s.sidecar_bytes
          << " ans_ratio=" << std::to_string(ans_ratio) << " disk_ratio=" << std::to_string(disk_ratio)
          << " owns_table=" << s.owns_table << " hist_ms=" << std::to_string(s.hist_ms)
          << " table_ms=" << std::to_string(s.table_ms) << " encode_ms=" << std::to_string(s.encode_ms)
          << " copy_ms=" << std::to_string(s.copy_ms) << " stored_bytes=" << s.stored_bytes
          << " unit_records=" << s.record_bytes << " slices=" << s.n_slices << "\n";
    }
    const std::string tag = "rank_" + std::to_string(std::max(c.rank, 0));
    o << lp << "[summary] tensors=" << written << " total_wall_ms=" << std::to_string(wall_ms)
      << " total_compute_ms=" << std::to_string(compute_ms) << " states=" << dir << "/" << tag << "_states.ansc"
      << " mantissa=" << dir << "/mantissa/" << tag << "_mantissa.mant tables=" << dir << "/tables/" << tag
      << "_tables.dict version=" << (unit ? 4 : 2) << "\n";
    o << "[TIMING] compress_and_save_total_ms=" << std::to_string(wall_ms) << "\n";
    o << "[TIMING] compress_computation_ms=" << std::to_string(compute_ms) << "\n";
    const std::string w(where);
    if (w == "stderr" || w == "1") {
        std::cerr << o.str() << std::flush;
    } else {
        std::ofstream f(w, std::ios::app);
        f << o.str();
    }
}

}  // namespace

void initialize_context(py::object model_engine, py::object optimizer, size_t histogram_bins,
                        size_t background_threads) {
    try {
        if (histogram_bins == 0) throw std::runtime_error("histogram_bins must be greater than zero");
        if (background_threads == 0) throw std::runtime_error("background_threads must be greater than zero");
        auto c = std::make_unique<Context>();
        c->rank = extract_rank(model_engine, "global_rank", "RANK");
        c->bins = histogram_bins;
        c->threads = background_threads;
        py::list named = py::module_::import("builtins").attr("list")(model_engine.attr("module").attr("named_parameters")());
        py::object opt = resolve_optimizer(model_engine, optimizer);
        if (!opt.is_none() && py::hasattr(opt, "fp16_partitioned_groups_flat") &&
            py::hasattr(opt, "fp32_partitioned_groups_flat")) {
            discover_zero3(*c, opt, named);
        } else {
            for (auto item : named) {
                py::tuple t = item.cast<py::tuple>();
                Record r;
                if (extract_tensor(t[1], c->rank, t[0].cast<std::string>(), &r)) c->recs.push_back(std::move(r));
                else c->skipped++;
            }
        }
        register_release_at_exit();
        release_context();  // the previous context's arena goes first
        place_records(*c, current_stream());
        // what analyze_tensors and compress_and_save will need, allocated now so
        // that neither allocates device memory (the reference plans its buffers
        // here too: compute_buffer_plan, MemoryManager.cpp:692-707)
        std::vector<ckr_device_tensor_record> recs;
        std::vector<ckr_ckpt_tensor> ts;
        for (const auto& r : c->recs) {
            recs.push_back(r.rec);
            if (r.rec.data_type == CKR_UNKNOWN) continue;
            ts.push_back(ckr_ckpt_tensor{r.name.c_str(), r.rec.d_ptr, r.rec.num_elements, r.rec.data_type, 0});
        }
        c->analyze_wsb = CKR(ckr_analyze_device_records_workspace_bytes)(recs.data(), recs.size());
        if (c->analyze_wsb && HIPFN(hipMalloc, void**, size_t)(&c->analyze_ws, c->analyze_wsb) != hipSuccess) {
            c->analyze_ws = nullptr;
            throw std::runtime_error("analyze workspace allocation failed");
        }
        check(CKR(ckr_ckpt_reserve)(ts.data(), ts.size(), unit_bytes_setting()), "checkpoint buffers");
        g_ctx = c.release();
    } catch (const std::exception& e) {
        throw std::runtime_error("[checkers] Context initialization failed: " + std::string(e.what()));
    }
}

void analyze_tensors() {
    try {
        if (!g_ctx) throw std::runtime_error("Context not initialized: MemoryManager logger is null.");
        Context& c = *g_ctx;
        if (c.recs.empty()) return;
        std::vector<ckr_device_tensor_record> recs;
        for (const auto& r : c.recs) recs.push_back(r.rec);
        void* stream = current_stream();
        const int rc = CKR(ckr_analyze_device_records)(recs.data(), recs.size(), c.analyze_ws, c.analyze_wsb, stream);
        std::vector<float> fp(recs.size() * 5, 0.f);
        hipError_t e = hipSuccess;
        for (size_t i = 0; i < recs.size() && rc == CKR_OK && e == hipSuccess; i++)
            e = HIPFN(hipMemcpyAsync, void*, const void*, size_t, hipMemcpyKind, hipStream_t)(&fp[i * 5], recs[i].d_fingerprint, 20, hipMemcpyDeviceToHost, (hipStream_t)stream);
        if (e == hipSuccess) e = HIPFN(hipStreamSynchronize, hipStream_t)((hipStream_t)stream);
        check(rc, "analyze");
        if (e != hipSuccess) throw std::runtime_error(std::string("fingerprint copy failed: ") + hip_error(e));
        // compute_fingerprint_weights (TensorAnalyzer.cpp:322-380); the reference
        // writes the weighted fingerprints back to the device, where nothing reads
        // them, and clusters the host copy (TensorAnalyzer.cpp:451)
        double weights[5];
        check(CKR(ckr_fingerprint_weights)(fp.data(), recs.size(), weights), "fingerprint weights");
        std::vector<const char*> names;
        for (const auto& r : c.recs) names.push_back(r.name.c_str());
        c.cluster_of.assign(recs.size(), -1);
        check(CKR(ckr_cluster)(names.data(), fp.data(), recs.size(), c.cluster_of.data(), nullptr), "clusters");
    } catch (const std::exception& e) {
        std::cerr << "[CHECKERS CRITICAL ERROR] " << e.what() << std::endl;
        throw;
    }
}

void compress_and_save(const std::string& output_path) {
    try {
        if (!g_ctx) throw std::runtime_error("Context not initialized: call initialize_context first.");
        Context& c = *g_ctx;
        const uint64_t unit = unit_bytes_setting();
        // CHECKERS_REPAIR_TABLES (default 1): a cluster table that the
        // reference's one-pass normalisation leaves above 4096 is repaired so that
        // its members can be decoded; 0 writes the reference's table unchanged
        int repair = 1;
        if (const char* v = std::getenv("CHECKERS_REPAIR_TABLES")) repair = std::atoi(v) != 0;
        std::vector<ckr_ckpt_tensor> ts;
        for (size_t i = 0; i < c.recs.size(); i++) {
            const Record& r = c.recs[i];
            if (r.rec.data_type == CKR_UNKNOWN) continue;  // no dtype tag: nothing the codec can size
            ckr_ckpt_tensor t{};
            t.name = r.name.c_str();
            t.d_ptr = r.rec.d_ptr;
            t.num_elements = r.rec.num_elements;
            t.dtype = r.rec.data_type;
            t.cluster_id = c.cluster_of.empty() ? -1 : c.cluster_of[i];
            ts.push_back(t);
        }
        std::vector<ckr_ckpt_stats> stats(std::max<size_t>(ts.size(), 1));
        const auto t0 = std::chrono::steady_clock::now();
        check(CKR(ckr_ckpt_write)(output_path.c_str(), std::max(c.rank, 0), ts.data(), ts.size(), unit, repair,
                                  stats.data(), current_stream()),
              "compress_and_save");
        const double wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        log_compress_stats(c, ts, stats, wall_ms, output_path, unit);
    } catch (const std::exception& e) {
        std::cerr << "[CHECKERS CRITICAL ERROR] compress_and_save: " << e.what() << std::endl;
        throw;
    }
}

}  // namespace checkers
