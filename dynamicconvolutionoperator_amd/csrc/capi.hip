// Library-level C-ABI helpers: status strings, ABI version, support queries,
// and the host-side launch helper shared by every entry point.
#include "gen_tile.h"

#include <map>
#include <mutex>
#include <utility>

namespace ddpm {

int allow_dynamic_lds(const void* fn, size_t bytes) {
  if (bytes <= 64 * 1024) return 0;  // the default limit
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> granted;  // (kernel, device) -> bytes
  std::lock_guard<std::mutex> lock(mu);
  size_t& have = granted[std::make_pair(fn, dev)];
  if (have >= bytes) return 0;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess) return (int)e;
  have = bytes;
  return 0;
}

}  // namespace ddpm

using namespace ddpm;

extern "C" int ddpm_abi_version(void) { return 7; }

extern "C" const char* ddpm_status_string(int code) {
  switch (code) {
    case kOk:
      return "ok";
    case kBadArgument:
      return "invalid argument (shape, kernel size, dilation, dtype or null pointer)";
    case kUnsupported:
      return "shape or kernel size not supported by this kernel";
    case kWorkspaceTooSmall:
      return "workspace missing or smaller than the entry point's *_workspace_bytes() query";
    case kScratchTooSmall:
      return "shape needs more scratch than the no-allocation entry point's fixed device buffer "
             "(ddpm_gen_bwd_y_noalloc_scratch_bytes())";
    default:
      return hipGetErrorString((hipError_t)code);
  }
}

// 1 when the fused generator kernels (forward and recompute backward) handle
// this channel count, kernel size and largest dilation, else 0 (the caller
// then materializes the dynamic kernels and uses the ddpm_filter_* entry
// points).  The backward kernels stage a column halo of kGenMaxDil pixels,
// and the 32-column tile's halo tile (16+2R) x (32+2R) pixels x 16 channels
// (fp32 entries, R = (K/2)*max_dilation) must fit the LDS of one workgroup
// next to two fp32 weight slices.
extern "C" int ddpm_gen_supported(int64_t c, int kernel_size, int max_dilation) {
  if (c < 1 || c > 128 || !(kernel_size == 1 || kernel_size == 3) || max_dilation < 1) return 0;
  if (kernel_size == 1) return 1;
  if (max_dilation > kGenMaxDil) return 0;
  GenGeom gg;
  if (gen_make_geom(gg, 1, c, 1, 1, kernel_size, max_dilation, max_dilation, max_dilation) != kOk)
    return 0;
  TileGeom g;
  size_t lds = 0;
  return tile_geom(g, gg, 16, 2, 2, lds) == kOk ? 1 : 0;
}

// 1 when the fused generator forward alone (inference: ddpm_gen_fwd) handles
// this channel count, kernel size (1, 3 or 5) and largest dilation, else 0:
// its halo tile of (16+2R) x (32+2R) pixels x 16 channels (fp32 entries, R =
// (K/2)*max_dilation) must fit the LDS of one workgroup next to two fp32
// weight slices and the bias rows.  At K <= 3 and dilations <= 8 this equals
// ddpm_gen_supported.
extern "C" int ddpm_gen_fwd_supported(int64_t c, int kernel_size, int max_dilation) {
  if (c < 1 || c > 128 || max_dilation < 1) return 0;
  if (!(kernel_size == 1 || kernel_size == 3 || kernel_size == kGenFwdMaxK)) return 0;
  if (kernel_size == 1) return 1;
  GenGeom gg;
  if (gen_make_geom(gg, 1, c, 1, 1, kernel_size, max_dilation, max_dilation, max_dilation,
                    kGenFwdMaxK) != kOk)
    return 0;
  TileGeom g;
  size_t lds = 0;
  return tile_geom(g, gg, 16, 2, 2, lds) == kOk ? 1 : 0;
}
