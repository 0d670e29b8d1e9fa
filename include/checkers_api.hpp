// checkers_api.hpp — the reference's C++ entry points (include/checkers/api.hpp:17-24,
// defined at src/api.cpp:899, :1033, :1255), kept with the same names,
// argument types and defaults, over this library's C ABI (checkers_amd.h).
// The pybind11 module `checkers_py` (checkers_amd/csrc/python_bindings.cpp)
// exposes exactly these three functions.  The reference header also declares
// analyze_model(), which it never defines; it is not declared here.
#ifndef CHECKERS_API_HPP
#define CHECKERS_API_HPP

#include <pybind11/pybind11.h>

#include <string>

namespace checkers {

namespace py = pybind11;

// Discover this rank's tensors (ZeRO-3 flat groups, else the model's named
// parameters), borrow their device memory, copy non-contiguous ones into the
// context's arena, and carve each tensor's statistics buffers from it.
// Errors: RuntimeError "[checkers] Context initialization failed: ...".
void initialize_context(py::object model_engine, py::object optimizer = py::none(), size_t histogram_bins = 256,
                        size_t background_threads = 1);

// Statistics pass, fingerprints, fingerprint weights and clusters.
void analyze_tensors();

// Compress every tensor and write rank_<r>_states.ansc, mantissa/rank_<r>_mantissa.mant
// and tables/rank_<r>_tables.dict under output_path.
void compress_and_save(const std::string& output_path);

}  // namespace checkers

#endif  // CHECKERS_API_HPP
