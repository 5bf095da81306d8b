// r4d_host.h -- host-side helpers of libr4d_mi355x: the error contract of the reference's C ABI
// (third_party/libr4d/r4d.h:30-31: an illegal shape throws std::runtime_error; the _check functions
// return nullptr or a message that stays valid until the calling thread's next check) and launch
// error reporting.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <stdexcept>
#include <string>

namespace r4d {

// The calling thread's last check message (what a _check entry returns a pointer to).
inline std::string& check_slot() {
  static thread_local std::string s;
  return s;
}
// nullptr for "", else the message kept in this thread's slot.
inline const char* check_result(const std::string& msg) {
  if (msg.empty()) return nullptr;
  check_slot() = msg;
  return check_slot().c_str();
}
[[noreturn]] inline void fail(const char* entry, const std::string& msg) {
  throw std::runtime_error(std::string("r4d ") + entry + ": " + msg);
}
inline void require(const char* entry, const std::string& msg) {
  if (!msg.empty()) fail(entry, msg);
}
inline void launch_ok(const char* entry) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(entry, std::string("launch failed: ") + hipGetErrorString(e));
}
// Lets kernel `fn` take up to 160 KiB of dynamic LDS on the current device (the attribute is per device): set once
// per device and kernel (`done` holds a bit per device, 64 at most), a failure thrown naming `entry`.
inline void allow_lds(const void* fn, std::atomic<unsigned long long>& done, const char* entry) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) fail(entry, "no usable current device");
  const unsigned long long bit = 1ull << dev;
  if (done.load(std::memory_order_acquire) & bit) return;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
    fail(entry, "hipFuncSetAttribute(MaxDynamicSharedMemorySize) failed");
  done.fetch_or(bit, std::memory_order_acq_rel);
}
inline bool pow2_in(int v, int lo, int hi) {
  return v >= lo && v <= hi && (v & (v - 1)) == 0;
}
inline std::string str(long long v) { return std::to_string(v); }

// The second pass of a split prefill launch (trellis_m256.hip): ws holds SKG fp32 slices [SKG][M][N];
// they are added in slice order, then full: FWHT-128 per column group (the reference's stage order), svh,
// out_scale, one bf16 rounding into C; else the fp32 sums into C. M a multiple of 32, N of 128.
void launch_split_finish(const float* ws, const float* svh, void* c, int M, int N, int SKG, int full, float out_scale,
                         hipStream_t st);

// Zeroes `bytes` bytes at p (4-byte aligned) with a fill kernel on st, ordered with the stream's other work and
// recordable in a HIP graph (no memset node); a launch failure thrown naming `entry`.
void launch_clear(void* p, size_t bytes, hipStream_t st, const char* entry);

}  // namespace r4d

// Arguments of one trellis GEMV launch (trellis_gemv.hip).
namespace r4d {
// The rule of the _parts entries' column starts: 1..4 parts, n0[0] = 0, rising in multiples of 128 below N.
inline std::string parts_rule(int parts, const int* n0, int N) {
  if (parts < 1 || parts > 4 || !n0) return "parts must be 1..4 with their first columns n0";
  if (n0[0] != 0) return "n0[0] must be 0";
  for (int p = 1; p < parts; ++p)
    if (n0[p] <= n0[p - 1] || n0[p] >= N || n0[p] % 128) return "n0 must rise in multiples of 128 below N";
  return "";
}
}  // namespace r4d

struct r4d_gemv_args {
  int64_t a0, a1;
  int n_split;
  int64_t w, svh, c, ws, tickets;
  int M, K, N, KB, SKG, full;
  float out_scale;
  int64_t stream;
  // the fused input transform (r4dx_trellis_gemv_xf / _xf_parts): xf = 1 for f16 x, 2 for bf16 x in a0; suh per
  // part (the parts' column starts as for the A parts below: n_split, n_end1, n_end2)
  int64_t suh0, suh1, suh2, suh3;
  int xf;
  float xscale;
  // SK = 1: one wave per tile pair over the whole K slice (the workgroup holds a 128-column group) also
  // when the launch is split -- the summation order r4d_gemm_trellis_nt_m256 reproduces
  int sk1;
  // the _raw entry's clock probe: 4 uint64 (shader clock, wall clock at entry; the same at the end of
  // workgroup (0, 0)'s own work), or 0
  int64_t clk;
  // the _wq measurement entries: the weight scale table [K / 16 >> wq_gsh][N] (0: off) and its group shift
  int64_t wsc;
  int wq_gsh;
  // more input parts (r4dx_gemm_trellis_nt_m64_parts): columns from n_end1 on read a2, from n_end2 on a3
  // (0: no such part)
  int64_t a2, a3;
  int n_end1, n_end2;
};

namespace r4d {
// Checks and launches one trellis GEMV (trellis_gemv.hip); throws std::runtime_error naming `entry` on an illegal
// launch.
void gemv_run(r4d_gemv_args& a, const char* entry);
}  // namespace r4d
