// checkers_amd/csrc/ckr_internal.h — shared between the kernels and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>

#include "checkers_amd.h"

namespace ckr {

// Table passed to kernels by value (1028 B of kernel arguments), so no host
// buffer has to outlive an asynchronous copy.  norm <= 4096 and cum <= 4096+256
// for every table normalize_histogram can produce, so 16 bits suffice.
struct TableArg {
    uint16_t norm[256];
    uint16_t cum[257];
};

// Per-symbol encode entry kept in LDS (16 B).  The division x/f of the
// reference's state update is replaced by a multiply-high with a per-symbol
// reciprocal (F. Giesen, "rans_byte.h", public domain, RansEncSymbolInit):
//   f >= 2: l = ceil(log2 f), rcp = ceil(2^(31+l)/f), rsh = l-1, bias = cum
//   f == 1: rcp = 2^32-1, rsh = 0, bias = cum + M - 1
//   q = mulhi(x, rcp) >> rsh == floor(x/f) for every x < 2^31
//   x' = x + bias + q*(M-f) == ((x/f) << 12) + cum + x%f
// xmax == 0 marks a symbol with f == 0 (the reference's raw-byte escape).
struct EncSym {
    uint32_t rcp;
    uint32_t bias;
    uint32_t cmpl_rsh;  // (M - f) | rsh << 16
    uint32_t xmax;      // 2^19 * f
};

// Decode slot entry: sym | (f-1) << 8 | cum << 20 (valid tables: f, cum < 4096).

// Optional per-kernel timing (ckr_profile_begin / ckr_profile_end): when on,
// every launch below is bracketed by HIP events recorded on its own stream.
void prof_mark(const char* name, hipStream_t s, bool begin);
// Whether ckr_profile_begin is in effect (launches are then timed one by one).
bool profiling();
extern thread_local bool t_noalloc;
// With profiling on, a device buffer of n u64 for per-unit phase stamps (else
// null); ckr_profile_end reduces the stamps of the last launch that used it.
uint64_t* prof_phase_buffer(uint64_t n, hipStream_t s);
#define CKR_LAUNCH(name, s, ...)              \
    do {                                      \
        ::ckr::prof_mark(name, s, true);      \
        __VA_ARGS__;                          \
        ::ckr::prof_mark(name, s, false);     \
    } while (0)
// Sets the calling thread's last error (ckr_last_error) and returns code.
int set_error(int code, const std::string& msg);

// ckr_encode_planes for a slice of a tensor whose own plane histograms are
// h_planes: every symbol of the slice is then known to have a slot, so the
// coders need no escape handling (ckr_encode_planes assumes escapes, since its
// histograms may belong to other data).  Same bytes either way.
int encode_slice_of_counted(const void* d_src, uint64_t n_elems, int dtype, const ckr_freq_table* h_table,
                            const uint32_t* h_planes, uint64_t unit_bytes, uint8_t* d_out, uint64_t out_capacity,
                            ckr_stream_header* d_headers, uint64_t* d_unit_offsets, uint8_t* d_sidecar,
                            void* d_workspace, uint64_t workspace_bytes, uint64_t* h_total_out, void* stream);

// ------------------------------------------------------------------ launchers
// All return hipError_t of the launch; geometry is decided inside.
hipError_t launch_build_enc_table(const TableArg& t, EncSym* d_enc, hipStream_t s);
// The encode entries and the fast encoder's status and control words cleared,
// in one launch (launch_encode_fast expects them).
hipError_t launch_build_enc_table_reset(const TableArg& t, EncSym* d_enc, uint64_t* status, uint64_t n_units,
                                        uint32_t* ctl, hipStream_t s);
// bad (may be null): a bad-lane counter to clear in the same launch.
hipError_t launch_build_dec_table(const TableArg& t, uint32_t* d_dec, unsigned long long* bad, hipStream_t s);

hipError_t launch_extract_mantissa(const uint8_t* src, uint64_t n_elems, int es, int spe,
                                   uint8_t* masked, uint8_t* sidecar, hipStream_t s);

// Masked histogram into d_hist[256] (overwritten); for masked dtypes, when
// d_planes is not null, d_planes[512] receives the two live planes' histograms.
// lean: a variant with 8 KiB of LDS per workgroup, which fits on a CU beside
// the fast encoder's workgroup, and one workgroup per CU (same counts).
uint32_t hist_num_blocks(uint64_t n_bytes);
// Several tensors' masked histograms (each with its live planes', 768 words at
// d_hists + 768 k, overwritten) in one grid per kMaxHistJobs of them.
struct HistSrc {
    const uint8_t* src;
    uint64_t n_bytes;
    int es, spe;
};
static constexpr uint32_t kMaxHistJobs = 16;
struct HistJob {
    const uint8_t* src;   // 16-byte aligned; the head_n bytes before it are the tensor's first
    uint64_t n_bytes;     // from src
    uint64_t zero_count;  // bytes of the masked planes, counted into bin 0 in closed form
    uint32_t* hist;       // 768 words
    uint32_t blk0, nblk, head_n;
    int32_t es, spe;
};
struct HistJobs {
    uint32_t n;
    HistJob j[kMaxHistJobs];
};
hipError_t launch_masked_hist_multi(const HistSrc* srcs, uint32_t n, uint32_t* d_hists, hipStream_t s);
// lean: the form that runs beside an encoder (4 copies per plane, one
// workgroup per CU); with chunk_ctr (a word of device memory, masked dtypes)
// its workgroups take chunks from that counter and the grid's others join in
// as the encoder leaves the CUs.
hipError_t launch_masked_hist(const uint8_t* src, uint64_t n_bytes, int es, int spe, uint32_t* d_hist,
                              uint32_t* d_planes, hipStream_t s, bool lean = false, uint32_t* chunk_ctr = nullptr);
// More workgroups (per_cu per CU) for a lean chunked histogram already queued
// with chunk_ctr: they take the chunks still left (none: they end at once).
hipError_t launch_masked_hist_join(const uint8_t* src, uint64_t n_bytes, int es, int spe, uint32_t* d_hist,
                                   uint32_t* d_planes, uint32_t* chunk_ctr, uint32_t per_cu, hipStream_t s);
hipError_t launch_set_u64(uint64_t* p, uint64_t v, hipStream_t s);
hipError_t launch_set_counter(unsigned long long* p, unsigned long long v, hipStream_t s);

// Encode one batch of units [u0, u0+nb).
struct EncodeGeom {
    uint64_t n_bytes;   // masked stream length n_b
    uint64_t unit;      // unit length U (multiple of 256, or n_b when single)
    uint64_t n_units;   // total units of the tensor
    uint32_t wmax;      // dword slots per lane in scratch
    int es, spe;
};
// ulist: when non-null, the batch is units ulist[u0 .. u0+nb) (offsets already
// known: no scan); otherwise units [u0, u0+nb).
hipError_t launch_encode_batch(const uint8_t* src, const EncodeGeom& g, uint64_t u0, uint64_t nb,
                               const EncSym* d_enc, const uint32_t* canon, uint32_t cw, bool dedup,
                               uint32_t* scratch, ckr_stream_header* hdrs, uint8_t* sidecar,
                               uint32_t* unit_size, uint64_t* unit_off, uint8_t* out, const uint32_t* ulist,
                               hipStream_t s);

// LDS-staged encode of all units (masked dtypes, units <= 64 KiB).  status:
// encode_fast_status_words(n_units) u64, ctl: 6 u32 ({ticket, redo count, error, 0, total lo, total hi}),
// both cleared beforehand by launch_build_enc_table_reset; redo_list: n_units u32 — units whose bytes
// must then be produced by launch_encode_batch.
struct FastEncParamsHost {
    uint32_t sl0, sl1, cw, canon_bytes;
    bool escapes;  // the data may hold symbols with f == 0 (table not built from it)
};
// LDS bytes of the fast encoder's workgroup within lds_limit (0: it does not fit).
uint32_t encode_fast_lds_bytes(const FastEncParamsHost& p, uint32_t lds_limit);
// The fast encoder's redo list (ctl[1] units) coded again: one coder pair per
// workgroup with slots that hold any lane; false/error when those slots do not
// fit lds_limit.
bool encode_fast_list_fits(const FastEncParamsHost& p, const EncodeGeom& g, uint32_t lds_limit);
hipError_t launch_encode_fast_list(const uint8_t* src, const EncodeGeom& g, const EncSym* d_enc, const uint32_t* canon,
                                   const FastEncParamsHost& hp, uint32_t lds_limit, ckr_stream_header* hdrs,
                                   uint8_t* out, uint64_t* unit_off, uint64_t* status, uint32_t* ctl,
                                   uint32_t* redo_list, hipStream_t s);
// Several tensors' fast encodes in one launch (same spe, sidecars for all or
// none, tables the data's own): each job's arguments as launch_encode_fast's,
// dsl its device slot sizes (sl0, sl1: the largest the launch's LDS holds);
// wg0 is set by the launcher.
struct FastJob {
    const uint8_t* src;
    EncodeGeom g;
    const EncSym* enc;
    const uint32_t* canon;
    ckr_stream_header* hdrs;
    uint8_t* sidecar;
    uint8_t* out;
    uint64_t* unit_off;
    uint64_t* status;
    uint32_t* ctl;
    uint32_t* redo;
    const uint32_t* dsl;
    uint32_t sl0, sl1, cw, canon_bytes;
    uint32_t wg0;
};
constexpr uint32_t kMaxFastJobs = 16;
struct FastJobs {
    uint32_t n;
    FastJob j[kMaxFastJobs];
};
hipError_t launch_encode_fast_multi(const FastJob* jobs, uint32_t n, uint32_t lds_limit, hipStream_t s);
// u64 look-back words of the fast encoder for n units (status argument size).
uint64_t encode_fast_status_words(uint64_t n_units);
// dsl (may be null): the two slot sizes in device memory (table_enc's tinfo +
// 258), used instead of hp's; hp's are then the largest the LDS holds.
hipError_t launch_encode_fast(const uint8_t* src, const EncodeGeom& g, const EncSym* d_enc, const uint32_t* canon,
                              const FastEncParamsHost& hp, uint32_t lds_limit, ckr_stream_header* hdrs,
                              uint8_t* sidecar, uint8_t* out, uint64_t* unit_off, uint64_t* status, uint32_t* ctl,
                              uint32_t* redo_list, hipStream_t s, const uint32_t* dsl = nullptr);
// Tables by ranks on the device (ckr_table.h): n histograms of 256 words into
// rows of 258 (norm_freq[256], sum, ambiguity flag).
hipError_t launch_tables(const uint32_t* hists, uint64_t n, int ensure_full, uint32_t* rows, hipStream_t s);
// A tensor's encode set-up from its histograms with no host round trip: table
// by ranks, encode entries, canonical zero-plane streams for lane counts k0,
// k1, k2 (cw dwords), the fast encoder's slot sizes (each at most smax, their
// sum at most 2 smax), and its status and control words cleared.  tinfo:
// norm[256], sum, ambiguity, sl0, sl1.
struct TableEncArg {
    uint32_t K, k0, k1, k2, cw, smax;
    int ensure_full;
};
struct TableEncJob {
    EncSym* enc;
    uint32_t* canon;
    uint32_t* tinfo;
    uint64_t* status;
    uint64_t n_status;
    uint32_t* ctl;
    TableEncArg a;
};
// Histogram words of an encode workspace (and of a device-table job): the 768
// of launch_masked_hist (all live bytes, plane FL, plane 3), then
// launch_hist_table's gate (768-769), done counter (770) and gate time-out
// stamp (772-773), and the lean histogram's chunk counter (776).
constexpr uint32_t kHistTableWords = 784;
// Masked histogram and table set-up of up to kMaxHistJobs tensors in one grid
// (launch_masked_hist_multi's shares): each job's first workgroup clears its
// histogram words and opens the job's gate with this launch's epoch, every
// workgroup adds its counts once the gate is open, and the job's last
// workgroup builds the table.  hist[j]: kHistTableWords words per job.
// epochs[j]: the epoch of job j's launch (written to its ctl[6..7] with the table).
// chains: the state chains of symbol 0 for every count (launch_canon_chains,
// kChainBytes, built once per device), from which the canonical streams are read.
hipError_t launch_hist_table(const HistSrc* srcs, uint32_t* const* hists, const TableEncJob* jobs, uint32_t n,
                             const void* chains, uint64_t* epochs, hipStream_t s);
constexpr uint32_t kChainRows = 4097;  // symbol-0 counts 0 .. 4096
constexpr uint32_t kChainSteps = 256;  // the most rows of a fast-encoder unit
constexpr uint64_t kChainBytes = (4ull + 2ull) * (kChainSteps + 1) * kChainRows + (2ull * kChainSteps + 8) * kChainRows;
hipError_t launch_canon_chains(void* chains, hipStream_t s);
constexpr uint32_t kTinfoWords = 260;
constexpr uint32_t kCanonMaxCw = 136;  // canonical stream dwords table_enc handles (K <= 256)
// The largest slot (multiple of 4, at most 2K + 8) whose two-pair layout of the
// fast encoder fits lds_cap (0: none).
uint32_t encode_fast_max_slot(uint32_t canon_bytes, uint32_t K, uint32_t lds_cap);

// Units above 64 KiB of masked dtypes, in two passes (no lane scratch): rec
// holds n_units * encode_seg_segments(unit) * 128 checkpoint records, unit_size
// n_units words, aux 128 words (aux[0]: nonzero when a segment did not end where
// its checkpoints say, which would be a bug).  With fp (slots sized for 256
// rows; units a multiple of 64 KiB), pass 2 runs on the fast encoder's waves,
// one 256-row segment per item, and seg_code_kernel takes the segments that do
// not fit the slots; ctl then holds 2 words and list
// encode_seg_list_items(n_units, unit) entries of 8 bytes.
uint32_t encode_seg_segments(uint64_t unit);
uint64_t encode_seg_list_items(uint64_t n_units, uint64_t unit);
// LDS bytes of pass 2 on the fast encoder's waves within lds_limit (0: it does not fit).
uint32_t encode_seg_fast_lds_bytes(const FastEncParamsHost& p, uint32_t lds_limit);
hipError_t launch_encode_seg(const uint8_t* src, const EncodeGeom& g, const EncSym* d_enc, const uint32_t* canon,
                             uint32_t cw, bool escapes, uint2* rec, ckr_stream_header* hdrs, uint32_t* unit_size,
                             uint64_t* unit_off, uint8_t* sidecar, uint8_t* out, uint32_t* aux,
                             const FastEncParamsHost* fp, uint32_t lds_limit, uint32_t* ctl, void* list,
                             hipStream_t s);

// Units above 1 MiB of masked dtypes (the one-stream layout of a large tensor,
// or large units), in two passes: one thread per lane chain records its state
// every LU_SEG rows, then every segment is coded side by side.  rec holds
// encode_long_rec_bytes(n_units, unit) bytes, unit_size n_units words, err one
// word (nonzero when a segment did not end at its record: a bug).
uint32_t encode_long_segments(uint64_t unit);
uint64_t encode_long_rec_bytes(uint64_t n_units, uint64_t unit);
hipError_t launch_encode_long(const uint8_t* src, const EncodeGeom& g, const EncSym* d_enc, bool escapes, uint2* rec,
                              ckr_stream_header* hdrs, uint32_t* unit_size, uint64_t* unit_off, uint8_t* sidecar,
                              uint8_t* out, uint32_t* err, hipStream_t s);
// Their decode: one block of four waves per unit, one lane chain per thread.
hipError_t launch_decode_long(const uint8_t* data, const ckr_stream_header* hdrs, const uint64_t* unit_off,
                              const uint32_t* d_dec, const EncodeGeom& g, const uint8_t* sidecar, uint8_t* dst,
                              unsigned long long* bad, hipStream_t s);

// Canonical zero-plane streams for lane counts k0, k1, k2: 3 entries of 4 + cw
// dwords (header, then the stream in slot format), followed by the 3 streams in
// byte order (cw dwords each).
// The same entries when the host has computed them, stored by small kernels
// whose argument carries n <= CANON_ARG_DWORDS of them, for canon[off .. off + n).
static constexpr uint32_t CANON_ARG_DWORDS = 900;
struct CanonArg {
    uint32_t n, off;
    uint32_t w[CANON_ARG_DWORDS];
};
hipError_t launch_canon_store(const CanonArg& a, uint32_t* canon, hipStream_t s);

// Several small tensors' fast decodes (ckr_decode_many): one set-up launch
// (each job's decode table from its frequency table staged in device memory,
// its canonical zero-plane streams from the state chains, its bad-lane counter
// cleared), then one decode launch over every job's units.
static constexpr uint32_t kMaxDecJobs = 16;
struct DecSetupJob {
    const TableArg* tab;   // staged in device memory
    uint32_t* dec;         // 4096 words
    uint32_t* canon;       // canonical streams (cw dwords per entry)
    unsigned long long* bad;
    uint32_t k0, k1, k2, cw;
};
struct DecSetupJobs {
    uint32_t n;
    DecSetupJob j[kMaxDecJobs];
};
struct DecJob {
    const uint8_t* data;
    const ckr_stream_header* hdrs;
    const uint64_t* unit_off;
    const uint32_t* dec;
    const uint32_t* canon;
    const uint8_t* sidecar;
    uint8_t* dst;           // 4-byte aligned
    unsigned long long* bad;
    EncodeGeom g;
    uint32_t cw, zero_bytes;
    uint32_t blk0, nblk;    // set by launch_decode_fast_multi
};
struct DecJobs {
    uint32_t n;
    DecJob j[kMaxDecJobs];
};
hipError_t launch_dec_setup_multi(const DecSetupJob* jobs, uint32_t n, const void* chains, hipStream_t s);
// Jobs of one spe (masked dtypes); hipErrorInvalidValue when they are not, or
// when the fast decoder's LDS does not fit the device (the caller then decodes
// them one by one).
hipError_t launch_decode_fast_multi(DecJob* jobs, uint32_t n, hipStream_t s);

// Decode; with canon (masked dtypes) the fast kernel decodes every unit,
// otherwise the general kernel does.
uint32_t decode_fast_lds_bytes();
// zero_bytes: the fast decoder also compares the zero-plane lanes' bytes with
// their canonical streams (their headers are checked either way); those bytes
// do not enter the output, so only a caller that reads the bad-lane count
// needs them read.
hipError_t launch_decode(const uint8_t* data, const ckr_stream_header* hdrs, const uint64_t* unit_off,
                         const uint32_t* d_dec, const EncodeGeom& g, const uint8_t* sidecar, uint8_t* dst,
                         unsigned long long* bad, const uint32_t* canon, uint32_t cw, hipStream_t s,
                         bool zero_bytes = true);

// Analyzer (ckr_analyzer.hip): every record in one grid per pass.
struct StatsParams {     // per record, device resident between passes
    float smin, smax, mean, scale;
    uint32_t use_range;  // range > 1e-9f
    uint32_t bins;
    uint32_t pad[2];
};
struct StatsPartial1 { float mn, mx; double sum; };
struct StatsPartial2 { double m2, m3, m4, pad; };
uint64_t analyze_workspace_bytes(const ckr_stats_record* recs, uint64_t n);
hipError_t launch_analyze(const ckr_stats_record* recs, uint64_t n, void* ws, hipStream_t s);

// Prefix-mask repair (ckr_repair.hip).
struct RepairCtl {
    uint64_t pick;        // tie-break: max of (bucket first occurrence << 32 | first occurrence)
    uint32_t n_cur, occ, done, round;  // live tokens; occurrences found this round
    uint32_t best, ncand, chosen, d;   // d: occupied pair-table slots
    uint32_t a0, a, b, c;              // alphabet size; pair (a, b) → c of this round
    uint32_t skip, tie, err, max_pair; // tie: several pairs hold the top count
    uint32_t recount, recount_next;    // build: count every pair this round / the next
    uint32_t run_mode;                 // a == b: occurrences depend on the run parity
    uint32_t pad[4];
};
constexpr uint32_t kRepairMaxPrimes = 512;
// Token ids of the repair sequence lie below these; the values from here up
// are tombstones (positions no live token holds) carrying span lengths.
constexpr uint32_t kRepairTomb16 = 0xF000u;
constexpr uint32_t kRepairTomb32 = 0xFFFF0000u;
struct RepairLayout {
    uint32_t w;           // live bits per word
    bool direct;          // w <= 16: alphabet by bitmap, else by hash set
    bool tok16;           // token ids (alphabet + rules) lie below kRepairTomb16
    uint64_t pair_cap, vcap, n_buckets, list_entries;
    uint32_t nids;        // bound of the token ids: alphabet (at most n, at most 2^w) + rules
    uint32_t hist_rows, hist_len;  // small alphabets: per-workgroup rows of count changes
    uint64_t o_ctl, o_tok, o_len, o_back, o_list, o_bcount, o_sym, o_bitmap, o_rank, o_vkey, o_vrank, o_occ;
    uint64_t o_pkey, o_pcnt, o_pfirst, o_touched, o_bfirst, o_primes, o_bfun, o_rules, o_rmap, o_hist;
    uint64_t bytes;
};
// n_buckets: bucket count of reserve(n) (size of the bucket first-occurrence array).
RepairLayout repair_layout(uint64_t n, int es, uint32_t k, uint32_t max_rules, uint64_t n_buckets);
struct RepairArgs {
    const uint8_t* words;
    uint64_t n;
    int es;
    uint32_t k;
    int build;                        // 1: build_shared_grammar, 0: apply rules
    uint32_t max_rules;
    const ckr_repair_rule* h_rules;   // apply: the rules
    uint32_t n_rules;
    const uint64_t* h_primes;         // build: library bucket counts covering [2, n], ascending
    uint32_t n_primes;
    uint64_t* d_seq_out;
    bool recount_each_round;          // build: every pair recounted each round
    uint8_t* ws;
    RepairLayout layout;
};
hipError_t repair_launch(const RepairArgs& a, hipStream_t s);

}  // namespace ckr
