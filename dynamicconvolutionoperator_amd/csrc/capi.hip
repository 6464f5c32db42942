// Library-level C-ABI helpers: status strings, ABI version, support queries,
// and the host-side launch helper shared by every entry point.
#include "gen_common.h"

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

extern "C" int ddpm_abi_version(void) { return 2; }

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
// and the forward's halo tile (16+2R) x (32+2R) pixels x 16 channels, R =
// (K/2)*max_dilation, must fit the 160 KB of LDS of one workgroup.
extern "C" int ddpm_gen_supported(int64_t c, int kernel_size, int max_dilation) {
  if (c < 1 || c > 64 || !(kernel_size == 1 || kernel_size == 3) || max_dilation < 1) return 0;
  if (kernel_size == 1) return 1;
  if (max_dilation > kGenMaxDil) return 0;
  const int64_t r = (int64_t)(kernel_size / 2) * max_dilation;
  const int64_t plane = ((16 + 2 * r) * (32 + 2 * r) * 4 * 4 + 255) / 256 * 256;
  const int64_t lds = 4 * plane + 2 * 2 * 2 * 64 * 16 + 3 * kernel_size * kernel_size * 16 * 4;
  return lds <= 160 * 1024 ? 1 : 0;
}
