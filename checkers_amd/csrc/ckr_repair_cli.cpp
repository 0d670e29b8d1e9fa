// checkers_amd/csrc/ckr_repair_cli.cpp — the tensor-group prefix-mask repair
// command line, with the grammar built and applied on the GPU through the C
// ABI (ckr_repair_build / ckr_repair_apply).
//
// Drop-in for the reference's CLI (src/tensor_group_prefix_mask_repair.cpp):
// same arguments (parse_args :606-640), same inputs (manifest.csv :219-249,
// analysis/plots/grouping_summary.csv :251-292, raw little-endian tensor files
// :294-326), same three reports under <export_dir>/prefix_mask_repair/
// (:477-604) with the same columns, formatting and size accounting (:642-731),
// and the same error texts and exit status (:744-754).  Only the time columns
// differ: they time this program.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <limits>
#include <map>
#include <optional>
#include <sstream>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "checkers_amd.h"

namespace {

namespace fs = std::filesystem;

struct Options {
    fs::path dir;
    size_t max_rules = 50;
    std::optional<std::string> state_type, category;
    std::optional<int> group_id;
    std::optional<size_t> masked_bits;
};

struct Tensor {
    std::string state_type, category, dtype;
    int layer = 0;
    size_t numel = 0;
    fs::path file;
};

struct Group {
    std::string state_type, category;
    int id = 0;
    std::vector<int> layers;
    int rep = 0;
};

struct Layout {          // storage bytes, mantissa bits, C-ABI tag
    size_t bytes, mantissa;
    int tag;
};

struct TensorRow {
    std::string state_type, category, dtype;
    int group_id = 0, layer = 0;
    bool rep = false;
    size_t numel = 0, masked_bits = 0, original = 0, masked_only = 0, tokens = 0, payload = 0, grammar = 0,
           residual = 0, lossy = 0, rules = 0;
    double mask_ratio = 1.0, ratio = 1.0, ms = 0.0;
};

struct GroupRow {
    std::string state_type, category, dtype;
    int id = 0, rep = 0;
    std::vector<int> layers;
    size_t masked_bits = 0, rules = 0, original = 0, masked_only = 0, payload = 0, grammar = 0, residual = 0,
           lossy = 0, max_pair = 0;
    double mask_ratio = 1.0, ratio = 1.0, ms = 0.0;
};

double ratio(double a, double b) { return std::abs(b) <= std::numeric_limits<double>::epsilon() ? 0.0 : a / b; }
double mb(size_t bytes) { return (double)bytes / (1024.0 * 1024.0); }
size_t bytes_of_bits(size_t bits) { return (bits + 7) / 8; }

// Smallest width that numbers `count` symbols (at least 1 bit).
size_t width_for(size_t count) {
    size_t w = 0;
    for (size_t v = count > 1 ? count - 1 : 0; v; v >>= 1) w++;
    return std::max<size_t>(w, 1);
}

Layout layout_of(const std::string& dt) {
    if (dt == "float32") return {4, 23, CKR_F32};
    if (dt == "float16" || dt == "fp16") return {2, 10, CKR_F16};
    if (dt == "bfloat16" || dt == "bf16") return {2, 7, CKR_BF16};
    throw std::runtime_error("Unsupported dtype for mantissa-mask compression: " + dt);
}

// CSV fields: double quotes toggle quoting and are dropped; each field is
// trimmed of spaces, tabs and CRs.
std::vector<std::string> split_csv(const std::string& line) {
    std::vector<std::string> out(1);
    bool quoted = false;
    for (char ch : line) {
        if (ch == '"') quoted = !quoted;
        else if (ch == ',' && !quoted) out.emplace_back();
        else out.back().push_back(ch);
    }
    for (auto& f : out) {
        const size_t a = f.find_first_not_of(" \t\r");
        f = a == std::string::npos ? std::string() : f.substr(a, f.find_last_not_of(" \t\r") - a + 1);
    }
    return out;
}

using Key = std::tuple<std::string, std::string, int>;

std::map<Key, Tensor> read_manifest(const fs::path& p) {
    std::ifstream in(p);
    if (!in) throw std::runtime_error("Failed to open manifest: " + p.string());
    std::string line;
    std::getline(in, line);  // header
    std::map<Key, Tensor> m;
    while (std::getline(in, line)) {
        if (line.empty()) continue;
        const auto c = split_csv(line);
        if (c.size() != 7) throw std::runtime_error("Malformed manifest row: " + line);
        Tensor t;
        t.layer = std::stoi(c[1]);
        t.category = c[2];
        t.state_type = c[3];
        t.numel = (size_t)std::stoull(c[4]);
        t.dtype = c[5];
        t.file = p.parent_path() / c[6];
        m[{t.state_type, t.category, t.layer}] = t;  // a later row replaces an earlier one
    }
    return m;
}

std::vector<Group> read_groups(const fs::path& p, const Options& o) {
    std::ifstream in(p);
    if (!in) throw std::runtime_error("Failed to open grouping summary: " + p.string());
    std::string line;
    std::getline(in, line);
    std::vector<Group> gs;
    while (std::getline(in, line)) {
        if (line.empty()) continue;
        const auto c = split_csv(line);
        if (c.size() < 10) throw std::runtime_error("Malformed grouping summary row: " + line);
        Group g;
        g.state_type = c[0];
        g.category = c[1];
        g.id = std::stoi(c[2]);
        std::istringstream ls(c[4]);
        for (int v; ls >> v;) g.layers.push_back(v);
        g.rep = std::stoi(c[5]);
        if ((o.state_type && g.state_type != *o.state_type) || (o.category && g.category != *o.category) ||
            (o.group_id && g.id != *o.group_id))
            continue;
        gs.push_back(std::move(g));
    }
    return gs;
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("[ckr] HIP error in ") + what + ": " + hipGetErrorString(e));
}
void ckr_check(int rc) {
    if (rc != CKR_OK) throw std::runtime_error(ckr_last_error());
}

// Device buffers that grow to the largest request.
struct DeviceBuf {
    void* p = nullptr;
    size_t cap = 0;
    void* get(size_t n) {
        if (n > cap) {
            if (p) hip_check(hipFree(p), "hipFree");
            p = nullptr;
            cap = 0;
            hip_check(hipMalloc(&p, std::max<size_t>(n, 256)), "hipMalloc");
            cap = std::max<size_t>(n, 256);
        }
        return p;
    }
    ~DeviceBuf() { if (p) (void)hipFree(p); }
};

// Reads the tensor file and copies it to the device; returns the device pointer.
void* load_to_device(const Tensor& t, const Layout& L, DeviceBuf& buf) {
    const size_t n = t.numel * L.bytes;
    std::vector<char> host(n);
    std::ifstream in(t.file, std::ios::binary);
    if (!in) throw std::runtime_error("Failed to open tensor payload: " + t.file.string());
    in.read(host.data(), (std::streamsize)n);
    if (in.gcount() != (std::streamsize)n) throw std::runtime_error("Tensor payload size mismatch: " + t.file.string());
    void* d = buf.get(n);
    if (n) hip_check(hipMemcpy(d, host.data(), n, hipMemcpyHostToDevice), "hipMemcpy");
    return d;
}

std::string join_layers(const std::vector<int>& v) {
    std::ostringstream s;
    for (size_t i = 0; i < v.size(); i++) s << (i ? " " : "") << v[i];
    return s.str();
}

void write_reports(const fs::path& dir, const std::vector<TensorRow>& trs, const std::vector<GroupRow>& grs,
                   const Options& o) {
    {
        std::ofstream f(dir / "tensor_prefix_mask_repair.csv");
        f << "state_type,category,group_id,layer,is_representative,dtype,numel,masked_mantissa_bits,"
             "original_size_mb,masked_only_size_mb,cfg_payload_size_mb,grammar_size_mb_charged,"
             "lossy_compressed_size_mb,residual_raw_size_mb,masking_only_ratio,compression_ratio,"
             "compressed_token_count,rule_count,time_ms\n";
        for (const auto& r : trs)
            f << r.state_type << ',' << r.category << ',' << r.group_id << ',' << r.layer << ',' << (r.rep ? 1 : 0)
              << ',' << r.dtype << ',' << r.numel << ',' << r.masked_bits << ',' << mb(r.original) << ','
              << mb(r.masked_only) << ',' << mb(r.payload) << ',' << mb(r.grammar) << ',' << mb(r.lossy) << ','
              << mb(r.residual) << ',' << r.mask_ratio << ',' << r.ratio << ',' << r.tokens << ',' << r.rules << ','
              << r.ms << '\n';
    }
    {
        std::ofstream f(dir / "group_prefix_mask_repair.csv");
        f << "state_type,category,group_id,layers,representative_layer,dtype,masked_mantissa_bits,rule_count,"
             "max_pair_frequency,original_group_size_mb,masked_only_group_size_mb,cfg_payload_group_size_mb,"
             "grammar_size_mb,lossy_compressed_group_size_mb,residual_raw_group_size_mb,masking_only_ratio,"
             "compression_ratio,total_time_ms\n";
        for (const auto& g : grs)
            f << g.state_type << ',' << g.category << ',' << g.id << ',' << '"' << join_layers(g.layers) << '"' << ','
              << g.rep << ',' << g.dtype << ',' << g.masked_bits << ',' << g.rules << ',' << g.max_pair << ','
              << mb(g.original) << ',' << mb(g.masked_only) << ',' << mb(g.payload) << ',' << mb(g.grammar) << ','
              << mb(g.lossy) << ',' << mb(g.residual) << ',' << g.mask_ratio << ',' << g.ratio << ',' << g.ms << '\n';
    }
    std::ofstream f(dir / "checkpoint_prefix_mask_repair_summary.txt");
    f << std::fixed << std::setprecision(6);
    f << "transform_mode: shared_group_mantissa_mask_cfg\n";
    f << "state_type_filter: " << (o.state_type ? *o.state_type : "<all>") << "\n";
    f << "category_filter: " << (o.category ? *o.category : "<all>") << "\n";
    f << "group_id_filter: ";
    if (o.group_id) f << *o.group_id; else f << "<all>";
    f << "\nmasked_mantissa_bits_request: ";
    if (o.masked_bits) f << *o.masked_bits; else f << "all_mantissa_bits";
    f << "\nmax_rules_shared_grammar: " << o.max_rules << "\n\n";
    size_t to = 0, tm = 0, tp = 0, tl = 0, tr = 0, tg = 0;
    for (const auto& g : grs) {
        to += g.original; tm += g.masked_only; tp += g.payload; tl += g.lossy; tr += g.residual; tg += g.grammar;
        f << g.state_type << '/' << g.category << "/group_" << g.id << ": layers=" << join_layers(g.layers)
          << ", representative_layer=" << g.rep << ", dtype=" << g.dtype << ", masked_mantissa_bits=" << g.masked_bits
          << ", rule_count=" << g.rules << ", original_group_size_mb=" << mb(g.original)
          << ", masked_only_group_size_mb=" << mb(g.masked_only) << ", cfg_payload_group_size_mb=" << mb(g.payload)
          << ", grammar_size_mb=" << mb(g.grammar) << ", lossy_compressed_group_size_mb=" << mb(g.lossy)
          << ", residual_raw_group_size_mb=" << mb(g.residual) << ", masking_only_ratio=" << g.mask_ratio
          << ", compression_ratio=" << g.ratio << '\n';
    }
    f << "\nselected_groups_original_size_mb: " << mb(to) << '\n';
    f << "selected_groups_masked_only_size_mb: " << mb(tm) << '\n';
    f << "selected_groups_cfg_payload_size_mb: " << mb(tp) << '\n';
    f << "selected_groups_total_grammar_mb: " << mb(tg) << '\n';
    f << "selected_groups_lossy_compressed_size_mb: " << mb(tl) << '\n';
    f << "selected_groups_residual_raw_size_mb: " << mb(tr) << '\n';
    f << "selected_groups_masking_only_ratio: " << ratio((double)to, (double)tm) << '\n';
    f << "selected_groups_compression_ratio: " << ratio((double)to, (double)tl) << '\n';
}

void run(const Options& o) {
    const auto manifest = read_manifest(o.dir / "manifest.csv");
    const auto groups = read_groups(o.dir / "analysis" / "plots" / "grouping_summary.csv", o);
    if (groups.empty()) throw std::runtime_error("No matching grouping rows found for the requested filters");
    const fs::path out = o.dir / "prefix_mask_repair";
    fs::create_directories(out);
    if (o.max_rules > 0xFFFFFFFFull) throw std::runtime_error("--max-rules too large");
    const int request = o.masked_bits ? (int)std::min<size_t>(*o.masked_bits, 64) : -1;

    DeviceBuf words, ws, rep_words;
    std::vector<TensorRow> trs;
    std::vector<GroupRow> grs;
    std::vector<ckr_repair_rule> rules(std::max<size_t>(o.max_rules, 1));
    for (const auto& g : groups) {
        const auto rit = manifest.find({g.state_type, g.category, g.rep});
        if (rit == manifest.end()) throw std::runtime_error("Missing representative tensor in manifest for requested group");
        const Tensor& rep = rit->second;
        const Layout L = layout_of(rep.dtype);
        const int k = ckr_repair_masked_bits(L.tag, request);
        size_t max_n = rep.numel;  // the workspace covers every tensor of the group
        for (int layer : g.layers) {
            const auto it = manifest.find({g.state_type, g.category, layer});
            if (it != manifest.end()) max_n = std::max(max_n, it->second.numel);
        }
        const uint64_t wsb = ckr_repair_workspace_bytes(max_n, L.tag, request, (uint32_t)o.max_rules);
        if (!wsb) throw std::runtime_error(ckr_last_error());
        void* dws = ws.get(wsb);
        void* drep = load_to_device(rep, L, rep_words);
        uint32_t nr = 0;
        uint64_t rep_tokens = 0, max_pair = 0;
        ckr_check(ckr_repair_build(drep, rep.numel, L.tag, request, (uint32_t)o.max_rules, rules.data(), &nr,
                                   &rep_tokens, &max_pair, nullptr, dws, wsb, nullptr));
        const size_t live = L.bytes * 8 - (size_t)k;
        const size_t width = width_for(((size_t)1 << live) + nr);
        const size_t grammar = bytes_of_bits(width * 2 * nr);

        GroupRow gr;
        gr.state_type = g.state_type; gr.category = g.category; gr.id = g.id; gr.layers = g.layers; gr.rep = g.rep;
        gr.dtype = rep.dtype; gr.masked_bits = (size_t)k; gr.rules = nr; gr.grammar = grammar; gr.max_pair = max_pair;
        bool charged = false;
        for (int layer : g.layers) {
            const auto it = manifest.find({g.state_type, g.category, layer});
            if (it == manifest.end()) throw std::runtime_error("Missing grouped tensor in manifest");
            const Tensor& t = it->second;
            if (t.dtype != rep.dtype) throw std::runtime_error("Mixed dtypes inside one group are not supported");
            const auto t0 = std::chrono::high_resolution_clock::now();
            const Layout Lt = layout_of(t.dtype);
            void* d = load_to_device(t, Lt, words);
            uint64_t tokens = rep_tokens;
            if (layer != g.rep)
                ckr_check(ckr_repair_apply(d, t.numel, Lt.tag, request, rules.data(), nr, &tokens, nullptr, dws, wsb,
                                           nullptr));
            TensorRow r;
            r.state_type = g.state_type; r.category = g.category; r.group_id = g.id; r.layer = layer;
            r.rep = layer == g.rep; r.dtype = t.dtype; r.numel = t.numel; r.masked_bits = (size_t)k;
            r.original = t.numel * Lt.bytes;
            r.masked_only = bytes_of_bits(t.numel * live);
            r.residual = bytes_of_bits(t.numel * (size_t)k);
            r.tokens = tokens;
            r.payload = bytes_of_bits(width * tokens);
            r.grammar = charged ? 0 : grammar;
            charged = true;
            r.lossy = r.payload + r.grammar;
            r.rules = nr;
            r.mask_ratio = ratio((double)r.original, (double)r.masked_only);
            r.ratio = ratio((double)r.original, (double)r.lossy);
            r.ms = std::chrono::duration<double, std::milli>(std::chrono::high_resolution_clock::now() - t0).count();
            gr.original += r.original; gr.masked_only += r.masked_only; gr.payload += r.payload;
            gr.residual += r.residual; gr.lossy += r.lossy; gr.ms += r.ms;
            trs.push_back(std::move(r));
        }
        gr.mask_ratio = ratio((double)gr.original, (double)gr.masked_only);
        gr.ratio = ratio((double)gr.original, (double)gr.lossy);
        grs.push_back(std::move(gr));
    }
    write_reports(out, trs, grs, o);
    std::cout << "Wrote tensor prefix-mask report to " << (out / "tensor_prefix_mask_repair.csv") << std::endl;
    std::cout << "Wrote group prefix-mask report to " << (out / "group_prefix_mask_repair.csv") << std::endl;
    std::cout << "Wrote prefix-mask summary to " << (out / "checkpoint_prefix_mask_repair_summary.txt") << std::endl;
}

Options parse(int argc, char** argv) {
    if (argc < 2)
        throw std::runtime_error(
            "Usage: tensor_group_prefix_mask_repair <export_dir> [--state-type NAME] [--category NAME] [--group-id N] "
            "[--max-rules N] [--masked-mantissa-bits N]");
    Options o;
    o.dir = argv[1];
    for (int i = 2; i < argc; i++) {
        const std::string a = argv[i];
        const bool has = i + 1 < argc;
        if (a == "--state-type" && has) o.state_type = std::string(argv[++i]);
        else if (a == "--category" && has) o.category = std::string(argv[++i]);
        else if (a == "--group-id" && has) o.group_id = std::stoi(argv[++i]);
        else if (a == "--max-rules" && has) o.max_rules = (size_t)std::stoull(argv[++i]);
        else if (a == "--masked-mantissa-bits" && has) o.masked_bits = (size_t)std::stoull(argv[++i]);
        else throw std::runtime_error("Unknown or incomplete argument: " + a);
    }
    return o;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        run(parse(argc, argv));
    } catch (const std::exception& e) {
        std::cerr << "tensor_group_prefix_mask_repair failed: " << e.what() << '\n';
        return 1;
    }
    return 0;
}
