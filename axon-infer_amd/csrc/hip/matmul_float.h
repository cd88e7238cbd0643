#pragma once

#include <cstdint>

namespace axon_hip {

// F32 / F16 / BF16 weights, or Q8_0 / Q4_0 / Q4_1 weights against float activations.
int matmul_float_launch(int type, const void* w, const float* x, float* y, uint32_t n_rows, uint32_t n_out,
                        uint32_t n_in, uint32_t y_stride);
// Per-block int32 sums of one weight row against one Q8_0 activation row (test hook).
int block_sums_launch(int type, const void* w_row, const void* xq, uint32_t n_blocks, int32_t* sumi, int32_t* sumx);

}  // namespace axon_hip
