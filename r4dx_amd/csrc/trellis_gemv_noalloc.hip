// trellis_gemv_noalloc.hip -- r4dx_gemm_trellis_nt_m64_noalloc: the trellis GEMV / skinny GEMM of
// trellis_gemv.hip with its split-K workspace and tickets in a library-held device array instead of caller
// buffers, for callers that cannot allocate (no reference counterpart).
#include "r4d_dev.h"
#include "r4d_host.h"
#include "r4d_mi355x.h"

#include <mutex>

// ---- the no-allocation form -------------------------------------------------------------------------------------
// No reference counterpart: r4d_gemm_trellis_nt_m64 for callers that cannot allocate or own a workspace (code under
// HIP graph capture, serving loops that forbid hipMalloc). The split partials and the tickets live in `scratch`, a
// file-scope device array of kNoAllocBytes per GPU that the library holds until the process ends: the first
// kNoAllocWsBytes take the partials [SKG][M][N] fp32, the rest the tickets (one 128-byte line per 128-column group,
// zero when the code object loads, cleared once more by a fill kernel at the first call on a device, and left zero
// by every complete launch). Every call on a GPU shares that GPU's array: calls that overlap on one GPU race.
namespace {
constexpr size_t kNoAllocWsBytes = (size_t)16 << 20;                          // partials: SKG * M * N * 4 at most
constexpr int kNoAllocMaxN = 262144;                                           // tickets for N up to this
constexpr size_t kNoAllocTicketBytes = (size_t)(kNoAllocMaxN / 128) * R4_TICKET_WORDS * 4;
constexpr size_t kNoAllocBytes = kNoAllocWsBytes + kNoAllocTicketBytes;
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

__global__ void noalloc_clear_kernel(unsigned* __restrict__ p, int words) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// The device address of this device's `scratch` (the host-side name of the array is not one), looked up once per
// device with that device current, its tickets cleared by a fill kernel on the caller's stream.
unsigned char* noalloc_scratch(hipStream_t st, const char* entry) {
  static std::mutex mu;
  static unsigned char* ptr[kNoAllocMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices) r4d::fail(entry, "no usable current device");
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) r4d::fail(entry, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    unsigned char* base = (unsigned char*)p;
    hipLaunchKernelGGL(noalloc_clear_kernel, dim3(64), dim3(256), 0, st, (unsigned*)(base + kNoAllocWsBytes),
                       (int)(kNoAllocTicketBytes / 4));
    r4d::launch_ok(entry);
    ptr[dev] = base;
  }
  return ptr[dev];
}
}  // namespace

extern "C" {

const char* r4dx_gemm_trellis_nt_m64_noalloc_check(int M, int K, int N, int n_split, int KB, int SKG) {
  if (const char* m = r4d_gemm_trellis_nt_m64_check(M, K, N, n_split, KB, SKG, 1, 1, 1)) return m;
  std::string e;
  if (N > kNoAllocMaxN) e = "N must be at most " + r4d::str(kNoAllocMaxN) + " (the scratch holds that many tickets)";
  else if (r4d_gemm_trellis_nt_m64_ws_bytes(M, N, SKG) > kNoAllocWsBytes)
    e = "SKG * M * N * 4 = " + r4d::str((long long)r4d_gemm_trellis_nt_m64_ws_bytes(M, N, SKG)) +
        " bytes of partials exceed the scratch's " + r4d::str((long long)kNoAllocWsBytes) + ": lower SKG or M";
  return r4d::check_result(e);
}

size_t r4dx_gemm_trellis_nt_m64_noalloc_max_ws_bytes(void) { return kNoAllocWsBytes; }

void r4dx_gemm_trellis_nt_m64_noalloc(int64_t a0, int64_t a1, int n_split, int64_t w, int64_t svh, int64_t c, int M,
                                      int K, int N, int KB, int SK, int SKG, float out_scale, int64_t stream) {
  const char* entry = "gemm_trellis_nt_m64_noalloc";
  if (const char* m = r4dx_gemm_trellis_nt_m64_noalloc_check(M, K, N, n_split, KB, SKG)) r4d::fail(entry, m);
  unsigned char* base = noalloc_scratch((hipStream_t)stream, entry);
  r4d_gemv_args a{a0, a1, n_split, w, svh, c, (int64_t)base, (int64_t)(base + kNoAllocWsBytes), M, K, N, KB, SKG, 1,
                  out_scale, stream};
  a.sk1 = SK == 1 || SK == 2;
  r4d::gemv_run(a, entry);
}

}  // extern "C"
