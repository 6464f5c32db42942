// Shape validation shared by the fused generator kernels (forward and backward).
#pragma once

#include "ddpm_common.h"

namespace ddpm {

struct GenGeom {
  int N, C, H, W, K;
  int d0, d1, d2;
  int R;        // halo radius (K/2)*max(d)
  int cblocks;  // ceil(C/16)
};

// Validates the shape for the fused kernels (odd K <= kmax: 3 for the
// recompute backward, 5 for the forward; C <= 128, dilations >= 1) and fills
// the geometry.  Returns kOk, kBadArgument or kUnsupported.
int gen_make_geom(GenGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int k, int d0, int d1,
                  int d2, int kmax = 3);

// Largest kernel size of the fused forward (inference; training at larger K
// materializes the kernels, as the reference's module does).
constexpr int kGenFwdMaxK = 5;

// Largest dilation the fused backward kernels stage (their column halo).
constexpr int kGenMaxDil = 8;

// Launches the split of an fp32 y [n][C][H*W] (chw = C*H*W elements per
// image, total = n*chw) into its bf16 hi / lo planes ys [n][2][C][H*W] on
// `stream`; returns the launch status.
int launch_ysplit(const float* y, uint16_t* ys, int64_t chw, int64_t total, hipStream_t stream);

}  // namespace ddpm
