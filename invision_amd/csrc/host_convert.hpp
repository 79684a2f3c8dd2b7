// host_convert.hpp -- fp32 -> bf16 rounding of host rows (host code only).
//
// Host fp32 operands that the device rounds to bf16 anyway (activations, Q, K,
// V) are rounded while they are copied into the pinned bounce buffers, so half
// the bytes cross PCIe.  The rounding is the device's bf16_rne bit for bit:
// nearest even, a NaN kept a NaN with its quiet bit set, overflow to infinity.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace inv {

// dst [rows x ldd] bf16 bits <- src [rows x lds] fp32, columns cols..cols_pad-1
// of each dst row zero.  One thread; AVX2 when the CPU has it.
void host_f32_to_bf16_rows(uint16_t *dst, int64_t ldd, const float *src, int64_t lds, int64_t rows, int64_t cols,
                           int64_t cols_pad);

}  // namespace inv
