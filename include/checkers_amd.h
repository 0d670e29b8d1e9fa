/*
 * checkers_amd.h — C ABI of the MI355X (gfx950) checkpoint-compression hot path.
 *
 * Every entry point takes plain pointers and sizes, returns an int status
 * (CKR_OK == 0, negative on error) and never throws; the message of the last
 * error on the calling thread is available from ckr_last_error().  Device
 * pointers ("d_" prefix) must be HIP device allocations on the current device;
 * host pointers ("h_" prefix) are ordinary host memory.  `stream` is a
 * hipStream_t passed as void* so that this header needs no HIP include.
 *
 * Reference interfaces replaced (paths relative to the reference tree):
 *   - ckr_extract_mantissa   ← extract_mantissa_kernel / ANSCompressor::extract_mantissa
 *                              (src/ANSCompressor.cpp:258-279, :945-1009)
 *   - ckr_byte_histogram     ← byte_histogram_kernel on the masked buffer
 *                              (src/ANSCompressor.cpp:109-126, launch :1225-1236)
 *   - ckr_byte_histogram_raw ← ANSCompressor::build_byte_histogram (src/ANSCompressor.cpp:393-411)
 *   - ckr_build_table        ← ANSCompressor::normalize_histogram (src/ANSCompressor.cpp:416-503)
 *   - ckr_build_table_ranked, ckr_build_tables_device ← the same, by ranks (host / device)
 *   - ckr_encode             ← rans_encode_kernel + compact_streams_kernel + the host prefix
 *                              sum and passthrough fallback of ANSCompressor::compress_tensor
 *                              (src/ANSCompressor.cpp:154-211, :225-238, :509-718)
 *   - ckr_decode             ← no counterpart: the reference has no decoder; this is the
 *                              inverse of rans_encode_kernel plus the sidecar merge
 *                              (include/checkers/ANSCompressor.hpp:165-171)
 *   - ckr_analyze            ← tensor_stats_kernel / compute_tensor_stats<T>
 *                              (src/TensorAnalyzer.cpp:64-229, launch :294-320), with the
 *                              fingerprint of TensorAnalyzer::compute_fingerprints
 *                              (src/TensorAnalyzer.cpp:271-292) written by the same pass
 *   - ckr_repair_build/apply ← build_shared_grammar / apply_existing_grammar of the
 *                              prefix-mask-repair CLI (src/tensor_group_prefix_mask_repair.cpp:328-467)
 */
#ifndef CHECKERS_AMD_H
#define CHECKERS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CKR_API __attribute__((visibility("default")))

/* ---- status codes ---- */
#define CKR_OK             0
#define CKR_E_INVALID    (-1)  /* bad argument (null pointer, size, dtype, unit) */
#define CKR_E_HIP        (-2)  /* a HIP runtime call failed                     */
#define CKR_E_CAPACITY   (-3)  /* caller-provided buffer too small              */
#define CKR_E_TABLE      (-4)  /* frequency table unusable for the operation    */
#define CKR_E_CORRUPT    (-5)  /* compressed stream failed a decode check       */

/* ---- dtype tags: include/checkers/TensorResource.hpp:30-37 ---- */
#define CKR_F32      0
#define CKR_BF16     1
#define CKR_F16      2
#define CKR_I8       3
#define CKR_I32      4
#define CKR_UNKNOWN  255

/* rANS constants: include/checkers/ANSCompressor.hpp:51-55 */
#define CKR_SCALE_BITS 12u
#define CKR_M          4096u
#define CKR_L          (1u << 23)
#define CKR_NORM_BASE  (1u << 19)
#define CKR_LANES      256u

/* Per-lane stream header: include/checkers/ANSCompressor.hpp:79-84 (16 bytes).
 * After ckr_encode, buf_offset is the lane's byte offset inside its chunk's
 * data (for a single-chunk tensor: inside the tensor's data, exactly as the
 * reference's compacted headers, src/ANSCompressor.cpp:685-691). */
typedef struct ckr_stream_header {
    uint32_t final_state;
    uint32_t byte_count;
    uint32_t buf_offset;
    uint32_t pad;
} ckr_stream_header;

/* Frequency table: include/checkers/ANSCompressor.hpp:64-74 (alignas(64), 40000 bytes). */
typedef struct __attribute__((aligned(64))) ckr_freq_table {
    uint32_t norm_freq[256];
    uint32_t cum_freq[257];
    uint32_t x_max[256];
    uint8_t  decode_sym[4096];
    uint32_t decode_freq[4096];
    uint32_t decode_cum[4096];
} ckr_freq_table;

/* Per-tensor analysis output (the three slab buffers of a DeviceTensorRecord,
 * include/checkers/MemoryManager.hpp:60-72; all device pointers, any may be NULL). */
typedef struct ckr_stats_record {
    const void* d_ptr;          /* tensor data                                  */
    uint64_t    num_elements;
    uint32_t    histogram_bins; /* clamped to 256 as in TensorAnalyzer.cpp:73    */
    uint32_t    data_type;      /* CKR_* tag                                    */
    uint32_t*   d_histogram;    /* [min(bins,256)] u32                          */
    float*      d_raw_moments;  /* [4] mean, var, skew, kurt                     */
    float*      d_minmax;       /* [2] min, max                                  */
    float*      d_fingerprint;  /* [5] mean, var, skew, kurt, max-min (or NULL)  */
} ckr_stats_record;

/* ---- library ---- */
CKR_API const char* ckr_last_error(void);
CKR_API const char* ckr_version(void);
/* Element size of a dtype tag (TensorResource.hpp:39-48); 0 for unknown tags. */
CKR_API int ckr_element_size(int dtype);
/* Low bytes moved to the sidecar per element (ANSCompressor.cpp:955-967): bf16/fp16 1, fp32 2, else 0. */
CKR_API int ckr_sidecar_bytes_per_elem(int dtype);

/* ---- byte-plane split (masked copy + element-interleaved sidecar) ---- */
CKR_API int ckr_extract_mantissa(const void* d_src, uint64_t n_elems, int dtype,
                                 void* d_masked, void* d_sidecar, void* stream);

/* ---- byte histogram of the masked byte stream, masking fused into the load.
 * d_hist[256] is overwritten (not accumulated).  For dtypes without a sidecar
 * the histogram is that of the raw bytes. ---- */
CKR_API int ckr_byte_histogram(const void* d_src, uint64_t n_elems, int dtype,
                               uint32_t* d_hist, void* stream);
/* Histogram of an arbitrary byte buffer (d_hist overwritten). */
CKR_API int ckr_byte_histogram_raw(const void* d_bytes, uint64_t n_bytes,
                                   uint32_t* d_hist, void* stream);
/* No counterpart in the reference (its tensors are encoded whole): the same
 * histogram into d_hist[0..256), and the histograms of the two live byte
 * planes (byte 2 or 1 of each 32-bit column, and byte 3) into d_hist[256..512)
 * and d_hist[512..768) (not written for dtypes without a sidecar).  With them,
 * ckr_encode_planes sizes the two-pass encoder's LDS slots when a large tensor
 * is encoded in slices under its whole-tensor table. */
CKR_API int ckr_byte_histogram_planes(const void* d_src, uint64_t n_elems, int dtype,
                                      uint32_t* d_hist, void* stream);

/* ---- host: histogram → table, same arithmetic and std::sort tie order as the
 * reference.  Returns CKR_OK; *h_table_sum receives sum(norm_freq) (4096 for a
 * valid table; larger in the reference's full-alphabet defect case, in which
 * the decode arrays are filled only up to slot 4095). ---- */
CKR_API int ckr_build_table(const uint32_t* h_hist, int ensure_full_alphabet,
                            ckr_freq_table* h_table, uint32_t* h_table_sum);

/* ---- the same table from ranks, on the host and on the device.  Replaces the
 * same normalize_histogram (src/ANSCompressor.cpp:416-503) without its sort:
 * each symbol's correction follows from how many fractional parts exceed or
 * equal its own.  That equals the sorted result unless the correction's
 * boundary falls inside a group of equal fractional parts, whose order only
 * libstdc++'s std::sort fixes: *h_ambiguous (or word 257 of a device row) is
 * then 1 and the caller must take ckr_build_table.  The device form builds
 * n tables from n histograms of 256 words (d_hists[i * 256 ..]) into n rows of
 * 258 words: norm_freq[256], their sum, the ambiguity flag. ---- */
CKR_API int ckr_build_table_ranked(const uint32_t* h_hist, int ensure_full_alphabet,
                                   ckr_freq_table* h_table, int* h_ambiguous);
CKR_API int ckr_build_tables_device(const uint32_t* d_hists, uint64_t n, int ensure_full_alphabet,
                                    uint32_t* d_rows, void* stream);

/* ---- chunked rANS encode ----
 * The masked byte stream of the tensor (n_b = n_elems * element_size bytes) is
 * cut into units of `unit_bytes` (a multiple of 256; unit_bytes >= n_b or 0
 * means one unit = the whole tensor, the reference layout).  Every unit is
 * coded exactly as rans_encode_kernel codes a whole tensor: 256 interleaved
 * lanes, each lane in reverse order, 12-bit table, byte renormalisation; the
 * lane streams are packed in lane order; a unit whose packed size is >= its
 * length is stored raw (the masked bytes; header 0 byte_count = length, all
 * other headers zero), the reference's passthrough rule applied per unit.
 * Outputs:
 *   d_out              packed data of all units, unit after unit;
 *   d_headers          n_units * 256 headers;
 *   d_unit_offsets     n_units + 1 u64: start of each unit's data in d_out,
 *                      the last entry is the total compressed size C;
 *   d_sidecar          sidecar bytes (n_elems * sidecar_bytes_per_elem) or NULL.
 * The table is given on the host.  The workspace must hold
 * ckr_encode_workspace_bytes(...) bytes; d_out must hold
 * ckr_encode_max_output_bytes(...) bytes.  If h_total_out is not NULL the
 * call synchronises `stream` and stores C there. ---- */
CKR_API uint64_t ckr_num_units(uint64_t n_elems, int dtype, uint64_t unit_bytes);
CKR_API uint64_t ckr_encode_max_output_bytes(uint64_t n_elems, int dtype, uint64_t unit_bytes);
CKR_API uint64_t ckr_encode_workspace_bytes(uint64_t n_elems, int dtype, uint64_t unit_bytes);
CKR_API int ckr_encode(const void* d_src, uint64_t n_elems, int dtype,
                       const ckr_freq_table* h_table, uint64_t unit_bytes,
                       uint8_t* d_out, uint64_t out_capacity,
                       ckr_stream_header* d_headers, uint64_t* d_unit_offsets,
                       uint8_t* d_sidecar,
                       void* d_workspace, uint64_t workspace_bytes,
                       uint64_t* h_total_out, void* stream);
/* No counterpart in the reference: ckr_encode with h_planes (host, 512 words:
 * d_hist[256..768) of ckr_byte_histogram_planes, for this data or for a tensor
 * it is a slice of), used only to size the encoders' LDS slots; the output is
 * ckr_encode's, byte for byte, whatever h_planes holds. */
CKR_API int ckr_encode_planes(const void* d_src, uint64_t n_elems, int dtype,
                              const ckr_freq_table* h_table, const uint32_t* h_planes,
                              uint64_t unit_bytes, uint8_t* d_out, uint64_t out_capacity,
                              ckr_stream_header* d_headers, uint64_t* d_unit_offsets,
                              uint8_t* d_sidecar, void* d_workspace, uint64_t workspace_bytes,
                              uint64_t* h_total_out, void* stream);

/* ---- full tensor compression as ANSCompressor::compress_tensor does it for a
 * singleton (histogram → table → encode), in one call.  The table built is
 * returned in h_table (may be NULL).  The workspace (16-byte aligned) as for
 * ckr_encode.  For tensors of masked dtypes with units of at most 64 KiB the
 * table is built on the device from the histogram in the same launch (the
 * reference's normalisation, by ranks; a table whose correction falls inside
 * a group of equal fractional parts is taken from the host's sort instead),
 * and the output buffers are checked while that launch runs: a bad output
 * buffer is reported once it has finished, with only the workspace written.
 * ---- */
CKR_API int ckr_compress(const void* d_src, uint64_t n_elems, int dtype, uint64_t unit_bytes,
                         int ensure_full_alphabet,
                         uint8_t* d_out, uint64_t out_capacity,
                         ckr_stream_header* d_headers, uint64_t* d_unit_offsets,
                         uint8_t* d_sidecar,
                         void* d_workspace, uint64_t workspace_bytes,
                         ckr_freq_table* h_table, uint64_t* h_total_out, void* stream);

/* ---- several tensors, as compress_and_save_all's workers take its items
 * (src/ANSCompressor.cpp:1118-1300, the GPU phases of each item): the same
 * results as ckr_compress called on each job in order, with job i+1's
 * histogram computed on a second, library-owned stream while job i is encoded,
 * the encodes alternating between `stream` and a third library-owned stream,
 * and the encodes queued back to back (each job's completion words are read
 * once, after the last).  When no job exceeds 256 MiB, every job's histogram
 * and table are built in one launch on the device instead and every encode of
 * one kind (dtype class, sidecar) in one more, with no host round trip between
 * them (tensors the device tables do not serve: every histogram first, one
 * host synchronisation, then the encodes round robin over four streams).
 * Every job has its own buffers and workspace (sizes as for ckr_compress).
 * Every job's sizes, source and workspace are checked before anything is
 * launched, its output buffers before anything writes them.  The inputs must
 * be ready in `stream` order; the call returns when every job is done, with
 * table and total filled in.  On error, jobs before the failing one are
 * complete. ---- */
typedef struct {
    const void* d_src;
    uint64_t n_elems;
    int32_t dtype;
    int32_t pad;
    uint8_t* d_out;
    uint64_t out_capacity;
    ckr_stream_header* d_headers;
    uint64_t* d_unit_offsets;
    uint8_t* d_sidecar;
    void* d_workspace;
    uint64_t workspace_bytes;
    ckr_freq_table* h_table;  /* filled (may be NULL) */
    uint64_t total;           /* filled: packed bytes */
} ckr_compress_job;
CKR_API int ckr_compress_many(ckr_compress_job* jobs, uint64_t n_jobs, uint64_t unit_bytes,
                              int ensure_full_alphabet, void* stream);

/* ---- decode: inverse of ckr_encode, sidecar merged back (original bits).
 * d_sidecar may be NULL only for dtypes without a sidecar.  The table must sum
 * to 4096.  Stream checks (every lane ends in state 2^23 having consumed
 * exactly byte_count bytes) are accumulated on the device; if h_bad_lanes is
 * not NULL the call synchronises and stores the number of failing lanes.  The
 * lanes of the masked (always zero) planes are checked against their
 * canonical stream, header and bytes; their bytes, which do not enter the
 * output, are read for that only when h_bad_lanes is not NULL. ---- */
CKR_API uint64_t ckr_decode_workspace_bytes(uint64_t n_elems, int dtype, uint64_t unit_bytes);
CKR_API int ckr_decode(const uint8_t* d_data, const ckr_stream_header* d_headers,
                       const uint64_t* d_unit_offsets,
                       const ckr_freq_table* h_table, uint64_t n_elems, int dtype,
                       uint64_t unit_bytes, const uint8_t* d_sidecar, void* d_dst,
                       void* d_workspace, uint64_t workspace_bytes,
                       uint64_t* h_bad_lanes, void* stream);

/* ---- several decodes in one call; no counterpart in the reference (it has
 * no decoder).  For restoring a shard: the same results as ckr_decode called
 * on each job.  When no job's output exceeds 256 MiB and the fast decoder
 * takes every non-empty job whole (masked dtypes, 4-byte aligned
 * destinations), every
 * job's set-up is one launch and every job's decode one more (per dtype
 * class), on `stream`; other small jobs go round robin over the caller's
 * stream and three library-owned streams, so that the decodes of small
 * tensors (too few units to fill the device) run side by side; larger jobs
 * alternate between `stream` and one library-owned stream, so that each
 * decode starts as the previous one's last units finish.
 * The inputs must be ready in
 * `stream` order, and the outputs are ready in `stream` order when the call
 * returns work queued (check == 0, no synchronisation).  check != 0: the call
 * synchronises and fills each job's bad_lanes.  Jobs share no destination or
 * workspace (sizes as for ckr_decode).  On error, the jobs before the failing
 * one are queued and complete in `stream` order. ---- */
typedef struct {
    const uint8_t* d_data;
    const ckr_stream_header* d_headers;
    const uint64_t* d_unit_offsets;
    const ckr_freq_table* h_table;
    uint64_t n_elems;
    int32_t dtype;
    int32_t pad;
    const uint8_t* d_sidecar;
    void* d_dst;
    void* d_workspace;
    uint64_t workspace_bytes;
    uint64_t bad_lanes;  /* filled when check != 0 */
} ckr_decode_job;
CKR_API int ckr_decode_many(ckr_decode_job* jobs, uint64_t n_jobs, uint64_t unit_bytes, int check,
                            void* stream);

/* ---- decode that allocates nothing; no counterpart in the reference.  For
 * callers that cannot allocate device memory: code under HIP graph capture,
 * serving loops that restore shards on the fly, harnesses that forbid
 * hipMalloc.  Same arguments and results as ckr_decode without the workspace:
 * the decoder's tables, canonical streams and bad-lane counter live in a
 * 128 KiB device array owned by the library, one per GPU, held until the
 * process ends (enough for every unit size up to 1 MiB and for the single-unit
 * layout; a larger need is CKR_E_CAPACITY).  The destination must be 4-byte
 * aligned (no staging copy is made).  Every call on a GPU uses that GPU's one
 * array, cleared by the call itself: calls that overlap on one GPU race, so
 * serialise them.  Under graph capture the call queues kernels only (the table
 * and canonical streams travel as kernel arguments); h_bad_lanes must then be
 * NULL (reading the count back synchronises; CKR_E_INVALID otherwise), and the
 * count stays in the scratch array until the next call. ---- */
CKR_API int ckr_decode_noalloc(const uint8_t* d_data, const ckr_stream_header* d_headers,
                               const uint64_t* d_unit_offsets,
                               const ckr_freq_table* h_table, uint64_t n_elems, int dtype,
                               uint64_t unit_bytes, const uint8_t* d_sidecar, void* d_dst,
                               uint64_t* h_bad_lanes, void* stream);

/* ---- TensorAnalyzer statistics pass over n records ----
 * All records go through four launches (two passes over the data, each with
 * every record's blocks in one grid).  The workspace size depends on each
 * record's pointer, element count and dtype (records with a null pointer, no
 * elements or an unknown dtype are skipped, as the reference skips them);
 * data pointers must be aligned to their element size. */
CKR_API uint64_t ckr_analyze_workspace_bytes(const ckr_stats_record* h_records, uint64_t n);
CKR_API int ckr_analyze(const ckr_stats_record* h_records, uint64_t n,
                        void* d_workspace, uint64_t workspace_bytes, void* stream);

/* ---- tensor-group prefix-mask repair (Re-Pair over masked words) ----
 * Replaces build_masked_sequence / find_best_pair / apply_rule /
 * build_shared_grammar / apply_existing_grammar of
 * src/tensor_group_prefix_mask_repair.cpp (:328-353, :376-467), the reference's
 * CPU-only CLI.  Words are the tensor's elements (F32, BF16 or F16) with their
 * low masked_bits mantissa bits cleared; masked_bits < 0 means all mantissa
 * bits (23, 7, 10), larger requests are clamped to them, as the reference does
 * (:333-336).  Rules are SharedGrammarRule (:70-75): rule i replaces the pair
 * (lhs, rhs) by the symbol 2^63 + i; symbols below 2^63 are masked words.
 * Ties between equally frequent pairs are broken as the reference's
 * std::unordered_map iteration order breaks them (libstdc++).  n_elems must be
 * below 2^31. ---- */
typedef struct {
    uint64_t replacement;
    uint64_t lhs;
    uint64_t rhs;
    uint64_t frequency;
} ckr_repair_rule;

/* Masked bit count the reference uses for a dtype and a request (<0: all
 * mantissa bits); -1 for a dtype the repair does not support. */
CKR_API int ckr_repair_masked_bits(int dtype, int request);
/* Bucket count of std::unordered_map::reserve(n) (libstdc++), the modulus of
 * the tie-break order; exported for tests. */
CKR_API uint64_t ckr_repair_bucket_count(uint64_t n);
CKR_API uint64_t ckr_repair_workspace_bytes(uint64_t n_elems, int dtype, int masked_bits, uint32_t max_rules);
/* build_shared_grammar on the tensor: up to max_rules rules into h_rules,
 * their count, the compressed token count and the largest pair count seen.
 * d_seq_out (n_elems u64, may be NULL) receives the compressed sequence as
 * reference symbols.  Synchronises `stream`. */
CKR_API int ckr_repair_build(const void* d_words, uint64_t n_elems, int dtype, int masked_bits,
                             uint32_t max_rules, ckr_repair_rule* h_rules, uint32_t* h_n_rules,
                             uint64_t* h_out_tokens, uint64_t* h_max_pair_frequency, uint64_t* d_seq_out,
                             void* d_workspace, uint64_t workspace_bytes, void* stream);
/* apply_existing_grammar: the rules in order, each a greedy left-to-right
 * pass.  Rule i must have replacement 2^63 + i.  Synchronises `stream`. */
CKR_API int ckr_repair_apply(const void* d_words, uint64_t n_elems, int dtype, int masked_bits,
                             const ckr_repair_rule* h_rules, uint32_t n_rules, uint64_t* h_out_tokens,
                             uint64_t* d_seq_out, void* d_workspace, uint64_t workspace_bytes, void* stream);

/* ---- fingerprint weights and clusters (host) ----
 * ckr_fingerprint_weights ← TensorAnalyzer::compute_fingerprint_weights
 * (src/TensorAnalyzer.cpp:322-380): h_fp holds n fingerprints of 5 floats
 * (mean, variance, skewness, kurtosis, range — what ckr_analyze writes);
 * h_weights[5] = per-dimension variance over the records / sum(variance + 1e-8).
 * ckr_cluster ← TensorAnalyzer::build_knn_clusters (:440-598): records are
 * grouped by name prefix ("optimizer.exp_avg_sq::", "optimizer.exp_avg::",
 * "master_weights::", else model state), fingerprints z-scored per category,
 * pairs closer than the lower quartile of all pairwise distances merged.
 * h_cluster_of[i] = cluster id (numbered per category in name order, then by
 * union-find root) or -1 for a singleton; h_threshold (optional, 4 doubles)
 * receives the merge threshold of each non-empty category in that order. */
CKR_API int ckr_fingerprint_weights(const float* h_fp, uint64_t n, double* h_weights);
CKR_API int ckr_cluster(const char* const* names, const float* h_fp, uint64_t n, int32_t* h_cluster_of,
                        double* h_threshold);

/* ---- rank checkpoint files ----
 * ckr_ckpt_write ← ANSCompressor::compress_and_save_all + write_rank_states_file /
 * write_rank_mantissa_file / write_rank_tables_file (src/ANSCompressor.cpp:1014-1401,
 * :721-931).  Tensors are taken in record order; those with a null pointer or
 * no elements are skipped.  cluster_id -1 (singleton) builds its own table;
 * the first compressed tensor of a cluster builds the cluster's table with the
 * full alphabet and the others reuse it (their anchor_name is the first record
 * of the cluster).  Writes <dir>/rank_<r>_states.ansc, <dir>/mantissa/
 * rank_<r>_mantissa.mant and <dir>/tables/rank_<r>_tables.dict.
 * unit_bytes 0: the reference's .ansc v2 (one stream per tensor, byte for byte
 * the reference's files; tensors must be below 4 GiB).  unit_bytes > 0: .ansc
 * v4, this library's chunked layout: header {magic, 4, rank, n, u64 unit_bytes,
 * u64 records_offset}, 576-byte index entries (the v2 entry without its
 * headers, then u64 n_units, u64 records offset, u64 records size), the stored
 * bytes of every tensor, then the unit records.  A unit record replaces the
 * unit's 256 lane headers: a raw unit is one byte; a coded unit keeps its live
 * lanes' final states (31 bits) and byte counts (as bit-packed deltas from the
 * least count of each byte plane), while the lanes of masked-out byte planes,
 * whose streams the table and the unit length determine, are stored neither
 * as headers nor as bytes (ckr_container.hip gives the exact layout).  Writes
 * stream: slice k+1 is encoded while slice k goes to the files through a
 * pinned host ring (16 x 32 MiB by default, CKR_CKPT_SLOTS; allocated on first
 * use and kept; calls serialise on it) and writer threads (CKR_CKPT_WRITERS).  repair_tables != 0 repairs a
 * full-alphabet table that the reference's one-pass normalisation leaves above
 * 4096 (such streams cannot be decoded) — a deliberate divergence, reported in
 * h_stats.  h_stats (optional) gets one entry per written tensor. */
typedef struct {
    const char* name;
    const void* d_ptr;
    uint64_t    num_elements;
    int32_t     dtype;
    int32_t     cluster_id;
} ckr_ckpt_tensor;

/* Per written tensor: the fields of the reference's per-tensor log line
 * (src/ANSCompressor.cpp:1292-1312) and its timing fields
 * (include/checkers/ANSCompressor.hpp:105-110): hist_ms = histogram and its
 * read-back, table_ms = host normalisation, encode_ms = encode launches until
 * the packed size is known, copy_ms = unit records and their read-back (the
 * file writes overlap the next encode and are not per tensor). */
typedef struct {
    uint64_t record_index;
    uint64_t original_bytes;
    uint64_t ans_bytes;      /* packed streams (unit records excluded)          */
    uint64_t sidecar_bytes;
    uint32_t owns_table;
    uint32_t table_sum;      /* sum of the table's frequencies (4096 unless the H1 case) */
    uint32_t table_repaired;
    uint32_t n_slices;       /* slices the tensor was encoded in                */
    uint64_t stored_bytes;   /* bytes of the tensor in the states file's data    */
    uint64_t record_bytes;   /* v4 unit records of the tensor                    */
    double   hist_ms, table_ms, encode_ms, copy_ms;
} ckr_ckpt_stats;

CKR_API int ckr_ckpt_write(const char* output_dir, int rank, const ckr_ckpt_tensor* tensors, uint64_t n,
                           uint64_t unit_bytes, int repair_tables, ckr_ckpt_stats* h_stats, void* stream);

/* The writer's device buffers (no counterpart in the reference, which sizes
 * its shared buffers for the largest tensor): a tensor is encoded in slices of
 * whole units under its whole-tensor table (units are independent streams
 * given the table, so the files are the same for any slice size), through two
 * buffer sets sized for one slice, kept from call to call.  The slice size is
 * CKR_CKPT_SLICE_BYTES (default 4 GiB) unless ckr_ckpt_set_slice_bytes set it
 * (0 returns to that default); a tensor that is one unit (v2) is one slice.
 * ckr_ckpt_reserve allocates the buffers and the pinned ring that
 * ckr_ckpt_write would need for these tensors, so that the write itself
 * allocates nothing; ckr_ckpt_write grows them when they are too small;
 * ckr_ckpt_pool_bytes reports the device bytes held; ckr_ckpt_release frees
 * all of it (also the pinned ring). */
CKR_API int ckr_ckpt_set_slice_bytes(uint64_t bytes);
CKR_API uint64_t ckr_ckpt_slice_bytes(void);
CKR_API int ckr_ckpt_reserve(const ckr_ckpt_tensor* tensors, uint64_t n, uint64_t unit_bytes);
CKR_API uint64_t ckr_ckpt_pool_bytes(void);
CKR_API void ckr_ckpt_release(void);

/* Reader (no counterpart in the reference): parses the three files of a rank
 * (v2 or v4 states file) and restores any tensor, bit-exact, into device
 * memory.  A tensor whose table does not sum to 4096 cannot be restored
 * (CKR_E_TABLE). */
typedef struct ckr_ckpt ckr_ckpt;
typedef struct {
    char     name[256];
    char     anchor_name[256];
    uint32_t dtype, is_raw, owns_table, version;
    uint64_t original_bytes, num_elements, data_size, n_units, unit_bytes, sidecar_bytes;
} ckr_ckpt_entry;
CKR_API int ckr_ckpt_open(const char* dir, int rank, ckr_ckpt** out);
CKR_API uint64_t ckr_ckpt_count(const ckr_ckpt* c);
CKR_API int ckr_ckpt_info(const ckr_ckpt* c, uint64_t index, ckr_ckpt_entry* out);
CKR_API int ckr_ckpt_restore(const ckr_ckpt* c, uint64_t index, void* d_dst, void* stream);
CKR_API void ckr_ckpt_close(ckr_ckpt* c);

/* ---- context memory: device records, arena, slabs, gather ----
 * ckr_device_tensor_record ← DeviceTensorRecord (include/checkers/MemoryManager.hpp:60-72),
 * the same 72-byte layout: the tensor's device pointer, its statistics buffers
 * carved from a slab, its element count, requested bins, dtype tag and
 * contiguity (0 contiguous, 1 non-contiguous, 2 scalar: TensorResource.hpp:53-57).
 * d_statistics is never set (the reference leaves it null as well). */
typedef struct ckr_device_tensor_record {
    const char* name;
    void*       d_ptr;
    uint32_t*   d_histogram;
    float*      d_raw_moments;
    void*       d_statistics;
    float*      d_fingerprint;
    float*      d_minmax;
    uint64_t    num_elements;
    uint32_t    histogram_bins;
    uint8_t     data_type;
    uint8_t     contiguity;
    uint8_t     pad_[2];
} ckr_device_tensor_record;

/* Arena: one hipMalloc of `capacity` bytes, handed out by bump allocation
 * (replaces the Umpire pools of MemoryManager / TensorResource,
 * src/MemoryManager.cpp:19-25, :403-425; src/TensorResource.cpp:38-55, :85-153).
 * ckr_arena_alloc returns CKR_E_CAPACITY when the arena is full; reset makes
 * all of it free again; destroy frees the device memory. */
typedef struct ckr_arena ckr_arena;
CKR_API int ckr_arena_create(uint64_t capacity, ckr_arena** out);
CKR_API int ckr_arena_alloc(ckr_arena* a, uint64_t bytes, uint64_t alignment, void** d_out);
CKR_API uint64_t ckr_arena_used(const ckr_arena* a);
CKR_API void ckr_arena_reset(ckr_arena* a);
CKR_API void ckr_arena_destroy(ckr_arena* a);

/* BufferPlan.total_bytes of one tensor (compute_buffer_plan,
 * src/MemoryManager.cpp:692-707): histogram (all requested bins, 4 bytes
 * each), 4 moments, min/max and the 5-float fingerprint, each rounded up to
 * `alignment` (the reference's default 256).  ckr_carve_stats_slab sets the
 * record's four buffer pointers in that order (the slab carving of
 * src/MemoryManager.cpp:440-466). */
CKR_API uint64_t ckr_stats_slab_bytes(uint32_t histogram_bins, uint64_t alignment);
CKR_API int ckr_carve_stats_slab(void* d_slab, uint32_t histogram_bins, uint64_t alignment,
                                 ckr_device_tensor_record* rec);
/* ckr_analyze over device records (their statistics buffers). */
CKR_API uint64_t ckr_analyze_device_records_workspace_bytes(const ckr_device_tensor_record* h_recs, uint64_t n);
CKR_API int ckr_analyze_device_records(const ckr_device_tensor_record* h_recs, uint64_t n, void* d_workspace,
                                       uint64_t workspace_bytes, void* stream);

/* make_contiguous ← TensorResource::make_contiguous (src/TensorResource.cpp:85-153):
 * copies a strided tensor (ndim <= 8, shape and strides in elements, element
 * size 1/2/4/8) into d_dst in row-major order.  The reference's fragments
 * (MemoryManager.cpp:709-740) assume rows with a unit inner stride; this
 * gather follows every stride, which is the same copy wherever that holds. */
CKR_API int ckr_make_contiguous(const void* d_src, int ndim, const int64_t* shape, const int64_t* strides,
                                int elem_size, void* d_dst, void* stream);

/* ---- path selection, no counterpart in the reference.  mode 1 (default):
 * fast kernels — lanes of masked planes coded once per lane count (their
 * streams are identical), units of at most 64 KiB coded and decoded through
 * LDS; mode 0: every lane coded and decoded independently through global
 * memory; mode 2: fast kernels with minimal LDS lane slots, so that nearly
 * every unit takes the overflow route back through the general kernels; mode
 * 3: the same minimal slots, the overflowing units coded again by the fast
 * encoder with slots that hold any lane (mode 1's overflow route).  In
 * mode 0 the prefix-mask repair build also recounts every pair each round
 * instead of keeping the counts up to date.  The output bytes are identical in
 * every mode; tests use this to cover all routes.  Process-wide; returns the
 * previous mode. ---- */
CKR_API int ckr_set_fast_paths(int mode);

/* ---- per-kernel timing, no counterpart in the reference (its only timings are
 * host wall clocks, ANSCompressor.hpp:105-110).  Between begin and end every
 * kernel the library launches is bracketed by HIP events on its stream; end
 * synchronises them and writes "<kernel> <launches> <total_ms>" lines.
 * Meanwhile ckr_compress_many and ckr_decode_many queue every encode and decode
 * on the caller's stream, so that each launch's events bracket its own kernel
 * and not one still running on another stream.  With
 * CKR_PROFILE_PHASES=1 in the environment the fast encoder also stamps each
 * unit's phases (extra work inside the kernel), reported as encode_fast.* lines. ---- */
CKR_API int ckr_profile_begin(void);
CKR_API int ckr_profile_end(char* buf, uint64_t buflen);

#ifdef __cplusplus
}
#endif
#endif /* CHECKERS_AMD_H */
