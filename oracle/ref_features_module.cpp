// Registers the reference's header-only CPU fused ops
// (python/src/features_bindings.hpp:336-382: fused.bias_gelu,
// fused.add_layernorm, ...) into a standalone Python module so the oracle can
// be checked against the reference's own C++ (built by `make ref` into
// oracle/_ref/). TEST INFRASTRUCTURE ONLY.
#include "features_bindings.hpp"

PYBIND11_MODULE(zref_features, m) {
  m.doc() = "reference CPU fused ops (checker build)";
  zenith::python::register_feature_bindings(m);
}
