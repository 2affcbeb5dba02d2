// Host-side staging rule of the streaming kernels, kept free of HIP headers
// so that it can be compiled and checked on its own.
#pragma once

#include <stdint.h>

namespace rbf {

// Whether the LDS-DMA kernels may stage an operand with n rows of d elements
// of esz bytes, rows stride_n elements apart.  The DMA reads each (b, h)
// slice through a buffer resource over [0, n * stride_n * esz) bytes whose
// size is a 32-bit field, and a row at an offset past that range reads as
// zeros.  So the rows must run forwards without overlapping (stride_n >= d:
// a zero stride -- a tensor expanded along N -- would make the range empty, a
// negative one would wrap the row offsets, and overlapping rows would put
// the last row's tail past the range), and the range must stay below 2^31.
// Operands that fail take the register-staged kernels, which index rows with
// signed 64-bit offsets.
inline bool dma_rows_ok(int64_t n, int64_t stride_n, int64_t d, int64_t esz) {
  if (n < 0 || d <= 0 || stride_n < d) return false;
  return n * stride_n * esz < (int64_t(1) << 31);
}

}  // namespace rbf
