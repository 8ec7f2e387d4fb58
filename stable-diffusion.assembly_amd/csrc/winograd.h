// Winograd's minimal filtering for 3x3 convolutions at stride 1
// (winograd.cc): F(2x2, 3x3) and F(4x4, 3x3), on the device.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/sdhip.h"
#include "device.h"

namespace sdhip {

struct WinogradArgs {
    int m;  // outputs of a tile along each side: 2 or 4
    const float *x;
    int64_t xnb1, xnb2, xnb3;
    int64_t iw, ih, ic, n;
    const _Float16 *w;    // [OC][IC][3][3] in FP16, or null
    const float *w32;     // the same in single precision, or null (F(2x2) only, winograd.cc:1204-1206)
    int64_t oc;
    float *y;
    int64_t ynb1, ynb2, ynb3;
    int64_t ow, oh;
    int32_t p0, p1;
    int64_t tw, th, tiles;  // tiles across, down, of all images
    int32_t from_redirect;
    DevChain chain;
    // Set by the launcher: the bytes of x from its first element past its
    // last where F(4x4)'s inputs can be read by rows of whole quads (see
    // winograd.hip), else 0; and the transformed inputs' layout, in runs of
    // 8 channels (1: [xi][part][kp / 8][tile][8], for the products whose
    // waves load their own rows) or of 32 (0: [xi][part][kp / 32][tile][32]).
    uint32_t xbytes;
    int32_t v_by8;
};

size_t winograd_work_size(const WinogradArgs &a);
sdhip_status winograd(const WinogradArgs &a, void *work, hipStream_t stream);

}  // namespace sdhip
