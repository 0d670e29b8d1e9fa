// checkers_amd/csrc/python_bindings.cpp — the `checkers_py` module: the three
// functions, argument names and defaults of the reference's module
// (src/python_bindings.cpp:17-34), defined by checkers_api.cpp.
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "checkers_api.hpp"

namespace py = pybind11;

PYBIND11_MODULE(checkers_py, m) {
    m.doc() = "Checkers checkpoint statistics and compression on MI355X (gfx950)";
    m.def("initialize_context", &checkers::initialize_context, py::arg("model_engine"),
          py::arg("optimizer") = py::none(), py::arg("histogram_bins") = 256, py::arg("background_threads") = 1,
          "Discovers this rank's tensors and places their statistics buffers in a device arena");
    m.def("analyze_tensors", &checkers::analyze_tensors,
          "Computes each tracked tensor's statistics, fingerprint and cluster");
    m.def("compress_and_save", &checkers::compress_and_save, "Compresses the tracked tensors and writes the rank's files");
}
