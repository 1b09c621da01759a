// layer_normalization challenge (reference adapter: tests/integration/layer_normalization.cu:3-4).
#include "adapter_common.hpp"

extern "C" void solve(const float *in, const float *gamma, const float *beta, float *out, int rows, int cols,
                      float eps) {
    opworks_adapter::guarded("layer_normalization",
                             [&] { opworks::ops::layer_norm(in, out, gamma, beta, rows, cols, eps); });
}
