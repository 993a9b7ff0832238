// Binds the reference's build_subgraph (csrc/cpu/subgraph.h, compiled from
// the reference tree by oracle/Makefile) as a Python module for parity tests.
// Test infrastructure only.
#include <torch/extension.h>

#include "cpu/subgraph.h"

PYBIND11_MODULE(ref_subgraph, m) {
  m.def("build_subgraph", &build_subgraph, "reference csrc/cpu/subgraph.cpp:8-114");
}
