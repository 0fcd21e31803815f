// Allocation-free variant of the int4 W4A16 GEMM.
//
// ti_w4a16_gemm takes a caller-owned split-K workspace.  Callers that cannot
// allocate device memory at all (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc) call ti_w4a16_gemm_noalloc instead:
// its split-K partial sums and tickets live in `scratch`, a file-scope device
// array of kScratchBytes that every GPU the library runs on holds until the
// process ends.  Nothing here calls hipMalloc, hipFree or an allocating
// library routine.
//
// In host code the name `scratch` is only a host-side stand-in for the array;
// its device address on the current GPU comes from hipGetSymbolAddress, taken
// once per device on the first call there and kept in g_scratch[device].  Only
// that address is handed to kernels.
//
// Every call on a GPU shares that GPU's array.  The split-K kernels leave the
// ticket words zero at the end of every call, and the array is zero-filled
// once at set-up, so each call starts from zero tickets; the partial sums are
// fully written before they are read.  Calls that overlap on one GPU (on
// different streams, or from different threads without ordering) race on the
// array and must not be issued.
#include <mutex>

#include "ti_common.h"

namespace ti {
namespace {

constexpr size_t kScratchBytes = 16u << 20;  // 16 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_lock;
void* g_scratch[kMaxDevices] = {};

__global__ __launch_bounds__(256) void zero_fill_kernel(uint4* __restrict__ p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Device address of this GPU's scratch array (set-up on first use: symbol
// lookup and a zero fill on `stream`).  Returns nullptr with the error set.
void* scratch_for_current_device(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("ti_w4a16_gemm_noalloc: no current HIP device (or device index >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch[dev]) return g_scratch[dev];
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) {
    set_error("ti_w4a16_gemm_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  hipLaunchKernelGGL(zero_fill_kernel, dim3(1024), dim3(256), 0, stream, (uint4*)ptr, kScratchBytes / 16);
  const hipError_t le = hipGetLastError();
  if (le != hipSuccess) {
    set_error("ti_w4a16_gemm_noalloc: scratch clear failed: %s", hipGetErrorString(le));
    return nullptr;
  }
  g_scratch[dev] = ptr;
  return ptr;
}

}  // namespace
}  // namespace ti

extern "C" size_t ti_w4a16_noalloc_scratch_bytes(void) { return ti::kScratchBytes; }

extern "C" int ti_w4a16_gemm_noalloc(const void* a, int dtype, const int32_t* packed_weight,
                                     const void* packed_scales, void* out, int M, int N, int K,
                                     int group_size, hipStream_t stream) {
  using namespace ti;
  const size_t need = ti_w4a16_workspace_bytes(M, N, K, group_size);
  if (need > kScratchBytes) {
    set_error("ti_w4a16_gemm_noalloc: problem M=%d N=%d K=%d needs %zu bytes of split-K scratch, "
              "more than the %zu-byte static buffer; call ti_w4a16_gemm with a workspace",
              M, N, K, need, kScratchBytes);
    return TI_ERR_WORKSPACE;
  }
  void* ptr = scratch_for_current_device(stream);
  if (!ptr) return TI_ERR_HIP;
  return ti_w4a16_gemm(a, dtype, packed_weight, packed_scales, out, M, N, K, group_size, ptr, kScratchBytes,
                       stream);
}
