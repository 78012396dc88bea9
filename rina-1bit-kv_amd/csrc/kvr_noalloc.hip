// kvr_decode_step_noalloc: kvr_decode_step for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The decode step's scratch -- the counter region, candidate lists, selected indices and
// partial records that kvr_decode_step takes as a caller-allocated workspace -- lives in
// the file-scope device array `scratch` below, KVR_NOALLOC_SCRATCH_BYTES (16 MiB) on every
// GPU the library runs on, held until the process ends.  Host code never passes the
// array's name to a kernel (in host code it is a host-side stand-in, not a device
// address): on the first call on a device, with that device current, the array's device
// address is looked up with hipGetSymbolAddress and kept per device, and the array is
// zeroed by a fill kernel on the caller's stream (the counter region must start at zero;
// calls leave it consistent for the next call).  That first call must not be under graph
// capture (a captured fill would zero the counters at every replay), so callers make one
// eager call first.  Nothing here calls hipMalloc, hipFree or an allocating library
// routine.
//
// Every call on a GPU shares that GPU's array: calls that overlap on one GPU (other
// streams, other threads) race and must be serialised by the caller.  The array's first
// int32 is the step's sticky status word (see kvr_decode_attn_workspace); a bounded wait
// that gives up shows as NaN outputs.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/kvr_capi.h"
#include "kvr_internal.h"

namespace {

constexpr size_t kScratchBytes = KVR_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ __launch_bounds__(256) void zero_scratch_kernel(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

std::mutex g_mu;
void* g_scratch[kMaxDevices];  // the device address of `scratch` on each device, once set up

// The scratch of the current device: looked up and zeroed on the device's first call.
int device_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return kvr::set_error(KVR_ERR_HIP, "kvr_decode_step_noalloc: no usable current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[dev]) {
    *out = g_scratch[dev];
    return KVR_OK;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
    return kvr::set_error(KVR_ERR_INVALID,
                          "kvr_decode_step_noalloc: the first call on device %d sets up its scratch and must not "
                          "be captured; make one call outside the capture first", dev);
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return kvr::set_error(KVR_ERR_HIP, "kvr_decode_step_noalloc: hipGetSymbolAddress failed: %s",
                          hipGetErrorString(e));
  hipLaunchKernelGGL(zero_scratch_kernel, dim3(1024), dim3(256), 0, stream, (uint4*)p, kScratchBytes / 16);
  if (hipError_t le = hipGetLastError())
    return kvr::set_error(KVR_ERR_HIP, "kvr_decode_step_noalloc: zeroing the scratch failed: %s",
                          hipGetErrorString(le));
  g_scratch[dev] = p;
  *out = p;
  return KVR_OK;
}

}  // namespace

extern "C" int kvr_decode_step_noalloc(const void* q, int q_dtype, int64_t B, int Hq, int Hkv, int d,
                                       const void* win_k, const void* win_v, int win_dtype, int64_t win_len,
                                       int64_t win_start, int64_t win_cap, int64_t win_stride_b,
                                       int64_t win_stride_h, int64_t win_stride_t, const uint64_t* kbits,
                                       const uint64_t* vbits, const uint16_t* kscale, const uint16_t* vscale,
                                       const uint8_t* kcounts, int64_t n_tiles, int64_t tile_stride, int T,
                                       int transform, const int32_t* excl_lo, const int32_t* excl_hi, int k,
                                       const int32_t* live_state, void* out, int out_dtype, int32_t* idx_out,
                                       kvr_stream_t stream) {
  const hipStream_t s = (hipStream_t)stream;
  // every check first (sizes beyond the scratch included): a rejected call launches nothing
  const size_t need = kvr::decode_step_workspace_bytes(B, Hq, Hkv, win_len, n_tiles, k, T);
  if (need > kScratchBytes)
    return kvr::set_error(KVR_ERR_WORKSPACE,
                          "kvr_decode_step_noalloc: these sizes need %zu bytes of scratch; the allocation-free "
                          "entry point holds %zu (use kvr_decode_step with a workspace)", need, kScratchBytes);
  if (int r = kvr::decode_step_impl(q, q_dtype, B, Hq, Hkv, d, win_k, win_v, win_dtype, win_len, win_start, win_cap,
                                    win_stride_b, win_stride_h, win_stride_t, kbits, vbits, kscale, vscale, kcounts,
                                    n_tiles, tile_stride, T, transform, excl_lo, excl_hi, k, live_state, out,
                                    out_dtype, idx_out, nullptr, kScratchBytes, s, false))
    return r;
  if (B == 0) return KVR_OK;
  void* ws = nullptr;
  if (int r = device_scratch(s, &ws)) return r;
  return kvr::decode_step_impl(q, q_dtype, B, Hq, Hkv, d, win_k, win_v, win_dtype, win_len, win_start, win_cap,
                               win_stride_b, win_stride_h, win_stride_t, kbits, vbits, kscale, vscale, kcounts,
                               n_tiles, tile_stride, T, transform, excl_lo, excl_hi, k, live_state, out, out_dtype,
                               idx_out, ws, kScratchBytes, s, true);
}
