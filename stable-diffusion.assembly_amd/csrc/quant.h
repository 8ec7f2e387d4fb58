// The quantized products of the reference's bits mode (sources/quant.h): the
// inputs unsigned with a zero point per (row, group of k), the weights signed
// and symmetric per (column, group) or per whole column, the products summed
// exactly in 32-bit integers and scaled back per group.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/sdhip.h"
#include "kernels.h"

namespace sdhip {

// The work buffer of a quantized MUL_MAT of K, N, M.
size_t quantized_linear_work_size(int64_t K, int64_t N, int64_t M);

// The quantized MUL_MAT (mul_mat.cc:498-569), or with `gated` the gated GELU
// after it (mul_mat.cc:577-646), of the product `a` describes.
sdhip_status quantized_linear(const MulMatArgs &a, bool gated, void *work, hipStream_t stream);

bool mul_mat_quantized(const sdhip_tensor *x);

// CONV_2D in the bits mode (quantize & 2): the direct convolution's products
// quantized (conv2d.cc:338-483), or, for the convolutions Winograd takes,
// F(2x2, 3x3) with quantized products (winograd.cc:1826-2103).  `c` as the
// direct convolution's (the kernel FP16 in w, or single precision in w32).
size_t quantized_conv_work_size(const ConvArgs &c, bool winograd);
sdhip_status quantized_conv(const ConvArgs &c, bool winograd, void *work, hipStream_t stream);

}  // namespace sdhip
