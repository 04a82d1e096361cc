// lsamp_noalloc.hip — lsamp_sample without a context, for callers that
// cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// The workspace the sampling kernels use (slice summaries, the row decisions,
// candidate and kept lists, per-chunk draw weights, arrival counters, the
// suppress bitmask) is a file-scope device array, `scratch`, laid out exactly
// as a context's (workspace_layout) for up to LSAMP_NOALLOC_MAX_ROWS rows of up
// to LSAMP_NOALLOC_MAX_VOCAB logits.  Each GPU holds its own copy for the
// life of the process.  In host code the array's name is only a stand-in:
// its device address on the current device comes from hipGetSymbolAddress,
// taken once per device on that device's first call and kept; every kernel
// argument uses that address.
//
// Every call on one GPU shares that GPU's array and leaves its contents
// behind: a call first clears the counters that must start at zero (a fill
// kernel, so the call can be captured in a HIP graph), and two calls that
// overlap on one GPU (different streams, no ordering) race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "lsamp_internal.h"

namespace lsamp {
namespace {

constexpr WorkspaceLayout kLayout =
    workspace_layout(LSAMP_NOALLOC_MAX_ROWS, LSAMP_NOALLOC_MAX_VOCAB);
static_assert(kLayout.total <= (size_t)LSAMP_NOALLOC_SCRATCH_BYTES,
              "the workspace fits the declared scratch size");
static_assert(kLayout.zero_end - kLayout.zero_begin <= 65536, "one small fill launch");

static __device__ __align__(256) unsigned char scratch[LSAMP_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

// What the first call on a device records (a fixed table: no allocation).
struct DeviceScratch {
  std::once_flag once;
  lsamp_status status = LSAMP_OK;
  char* ptr = nullptr;  // the device address of `scratch` on this device
  DeviceShape shape{};
  WorkspaceViews views{};
};
DeviceScratch g_devices[kMaxDevices];

void setup_device(DeviceScratch& d, int device) {
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
    d.status = LSAMP_ERR_DEVICE;
    return;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus <= 0) {
    d.status = LSAMP_ERR_DEVICE;
    return;
  }
  d.ptr = static_cast<char*>(ptr);
  d.shape = query_device_shape(cus);
  d.views = bind_workspace(d.ptr, LSAMP_NOALLOC_MAX_ROWS, LSAMP_NOALLOC_MAX_VOCAB);
}

__global__ __launch_bounds__(256) void k_zero_words(uint32_t* p, int32_t n) {
  const int32_t i = (int32_t)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) p[i] = 0u;
}

}  // namespace

int launch_zero_words(void* p, size_t bytes, void* stream) {
  const int32_t n = (int32_t)(bytes / 4);
  hipLaunchKernelGGL(k_zero_words, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<uint32_t*>(p), n);
  return (int)hipGetLastError();
}

}  // namespace lsamp

using namespace lsamp;

extern "C" lsamp_status lsamp_sample_noalloc(const lsamp_sample_args* a, void* stream) {
  if (!a) return set_error(LSAMP_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->rows > LSAMP_NOALLOC_MAX_ROWS || a->vocab > LSAMP_NOALLOC_MAX_VOCAB)
    return set_error(LSAMP_ERR_CAPACITY,
                     "rows %d / vocab %d exceed the no-allocation limits (%d rows, %d vocab)",
                     a->rows, a->vocab, LSAMP_NOALLOC_MAX_ROWS, LSAMP_NOALLOC_MAX_VOCAB);
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices)
    return set_error(LSAMP_ERR_DEVICE, "no usable current device (%d)", device);
  DeviceScratch& d = g_devices[device];
  std::call_once(d.once, setup_device, std::ref(d), device);
  if (d.status != LSAMP_OK)
    return set_error(d.status, "the scratch workspace of device %d is not available", device);
  // the step's counters start at zero whatever an earlier call left
  const int err = launch_zero_words(d.views.zero_begin, d.views.zero_bytes, stream);
  if (err != 0)
    return set_error(LSAMP_ERR_DEVICE, "kernel launch failed: %s",
                     hipGetErrorString((hipError_t)err));
  lsamp_launch_info last{};
  return sample_step(d.views, d.shape, LSAMP_MODE_AUTO, a, stream, nullptr, &last);
}
