// checkers_amd/csrc/ckr_container.h — unit records of the chunked states file
// (.ansc v4): device pack on the writer's side, host expansion on the reader's.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "checkers_amd.h"

namespace ckr {

struct UnitGeomArg {
    uint64_t n_bytes;  // masked stream length of the tensor
    uint64_t unit;     // unit length (multiple of 256)
    uint64_t n_units;
    int es, spe;       // element size; sidecar bytes per element (zero-plane residues 0..spe-1)
};

// Zero-plane lane streams for the three lane symbol counts a tensor's units
// have: k[0] (full units), k[1], k[2] (the last unit: ceil and floor of len/256).
struct ZeroLaneArg {
    uint32_t k[3], state[3], count[3];
};
struct ZeroLanes {
    ZeroLaneArg arg;
    std::vector<uint8_t> bytes[3];  // each stream in stored (data) order
};
ZeroLanes zero_lanes(const ckr_freq_table* t, uint64_t n_bytes, uint64_t unit);
uint32_t zero_lane_stream(const ckr_freq_table* t, uint32_t K, std::vector<uint8_t>* bytes);

constexpr uint32_t kUnitRecordMax = 1 + 256 * 8;  // the largest unit record (kind 2)

// Per unit: the record's size and the number of its bytes that are stored.
hipError_t launch_unit_plan(const ckr_stream_header* hdr, const UnitGeomArg& g, const ZeroLaneArg& z,
                            uint32_t* rec_size, uint32_t* data_size, hipStream_t s);
// Records to rec_out + rec_off[u], stored bytes to data_out + out_off[u].
hipError_t launch_unit_pack(const uint8_t* data, const uint64_t* unit_off, const ckr_stream_header* hdr,
                            const UnitGeomArg& g, const ZeroLaneArg& z, const uint64_t* rec_off,
                            const uint64_t* out_off, uint8_t* rec_out, uint8_t* data_out, hipStream_t s);

// A tensor's records and stored bytes back to the 256 headers per unit, the
// unit offsets and the units' full data, as the encoder wrote them.  Returns
// CKR_OK or CKR_E_CORRUPT with the reason in why.
int expand_units(const uint8_t* rec, uint64_t rec_size, const uint8_t* stored, uint64_t stored_size,
                 uint64_t n_bytes, uint64_t unit, int es, int spe, const ZeroLanes& z,
                 std::vector<ckr_stream_header>& hdr, std::vector<uint64_t>& uoff, std::vector<uint8_t>& data,
                 std::string& why);

}  // namespace ckr
