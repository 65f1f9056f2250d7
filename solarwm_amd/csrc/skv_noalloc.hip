// skv_attention_ex_noalloc: skv_attention_ex for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops).  The balanced key split keeps its
// partial results in a file-scope device array instead of a caller workspace.  The array lives
// in this translation unit's own code object, so a process that never calls this entry point
// never loads it; a process that does holds it on every GPU it calls from until it exits.
#include <mutex>

#include "skv_common.h"

namespace {

// Partial-result records of the split: 2 per workgroup (one workgroup per CU) of 256 query
// rows x (128 O floats + running max + row sum).  Sized for 256 CUs (MI355X): 68,157,440 B.
constexpr int kScratchCus = 256;
constexpr int64_t kScratchBytes = (int64_t)2 * kScratchCus * 256 * (128 + 2) * sizeof(float);
static_assert(kScratchBytes == SKV_NOALLOC_SCRATCH_BYTES, "header constant out of date");

__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};  // device address of `scratch` on each device

// The device address of this device's copy of `scratch`, looked up once per device with that
// device current (host code never uses the array's name as an address).  The first lookup on a
// device loads this file's code object there (deferred loading) and places the array, which a
// stream under graph capture must not do: with `stream` capturing and no address known yet the
// call fails and names skv_noalloc_init, which callers make once per device before capturing.
int scratch_ptr(void** out, skv_stream_t stream, bool from_init) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    skv::set_error("%s: no usable current device (%s)",
                   from_init ? "skv_noalloc_init" : "skv_attention_ex_noalloc",
                   e != hipSuccess ? hipGetErrorString(e) : "device index out of range");
    return SKV_E_LAUNCH;
  }
  std::lock_guard<std::mutex> g(g_mu);
  if (!g_scratch[dev] && !from_init) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs) == hipSuccess &&
        cs != hipStreamCaptureStatusNone) {
      skv::set_error("skv_attention_ex_noalloc: the scratch array of device %d is not set up; "
                     "call skv_noalloc_init() with that device current before capturing", dev);
      return SKV_E_UNSUPPORTED;
    }
  }
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      skv::set_error("skv_attention_ex_noalloc: hipGetSymbolAddress of the scratch array "
                     "failed on device %d: %s", dev, hipGetErrorString(e));
      return SKV_E_LAUNCH;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return SKV_OK;
}

}  // namespace

extern "C" int skv_attention_ex_noalloc(const skv_attention_desc* d, skv_stream_t stream) {
  skv::clear_error();
  if (!d) {
    skv::set_error("skv_attention_ex_noalloc: null descriptor");
    return SKV_E_ARG;
  }
  if (d->workspace || d->workspace_bytes) {
    skv::set_error("skv_attention_ex_noalloc: uses its own static scratch; pass workspace = NULL "
                   "and workspace_bytes = 0 (or call skv_attention_ex with a workspace)");
    return SKV_E_ARG;
  }
  skv_launch_plan plan;
  int st = skv::attention_with_workspace(d, nullptr, 0, nullptr, &plan);
  if (st != SKV_OK) return st;
  if (plan.workspace_bytes > kScratchBytes) {
    skv::set_error("skv_attention_ex_noalloc: this launch needs %lld bytes of scratch, more than "
                   "the static %lld (sized for %d CUs)", (long long)plan.workspace_bytes,
                   (long long)kScratchBytes, kScratchCus);
    return SKV_E_UNSUPPORTED;
  }
  void* ws = nullptr;
  if (plan.workspace_bytes > 0) {
    st = scratch_ptr(&ws, stream, false);
    if (st != SKV_OK) return st;
  }
  return skv::attention_with_workspace(d, ws, ws ? kScratchBytes : 0, stream, nullptr);
}

extern "C" int skv_noalloc_init(void) {
  skv::clear_error();
  void* p = nullptr;
  return scratch_ptr(&p, nullptr, true);
}
