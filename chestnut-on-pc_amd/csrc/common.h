// Shared definitions for the chestnut gfx950 library: error convention,
// vector types, wave-level reductions and the image2d texel addressing rule.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace ck {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

void set_last_error(const std::string& msg);

#define CK_HIP(call)                                                                 \
  do {                                                                               \
    hipError_t e_ = (call);                                                          \
    if (e_ != hipSuccess)                                                            \
      throw ::ck::Error(std::string(#call) + " failed: " + hipGetErrorString(e_));   \
  } while (0)

#define CK_REQUIRE(cond, msg)                                                        \
  do {                                                                               \
    if (!(cond)) throw ::ck::Error(std::string(msg));                                \
  } while (0)

// Launch check: a launch error (bad grid, invalid symbol) surfaces here.
#define CK_LAUNCHED(what) CK_HIP(hipGetLastError())

// In-frame kernel timing.  While `on` is set on this thread (eager launches
// only, never under graph capture), every CK_LAUNCH goes through
// hipExtLaunchKernelGGL with a start and a stop event, which receive the
// dispatch's own begin and end timestamps -- the interval a kernel trace
// reports, with no marker packet between the frame's kernels.  The caller
// owns and destroys the recorded events.
struct LaunchTimer {
  bool on = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> events;
};
LaunchTimer& launch_timer();

#define CK_LAUNCH(kernel, grid, block, shmem, stream, ...)                                      \
  do {                                                                                          \
    ::ck::LaunchTimer& ck_lt_ = ::ck::launch_timer();                                           \
    if (ck_lt_.on) {                                                                            \
      hipEvent_t ck_e0_ = nullptr, ck_e1_ = nullptr;                                            \
      CK_HIP(hipEventCreate(&ck_e0_));                                                          \
      ck_lt_.events.emplace_back(ck_e0_, nullptr);                                              \
      CK_HIP(hipEventCreate(&ck_e1_));                                                          \
      ck_lt_.events.back().second = ck_e1_;                                                     \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, ck_e0_, ck_e1_, 0, __VA_ARGS__); \
    } else {                                                                                    \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                      \
    }                                                                                           \
  } while (0)

typedef _Float16 half_t;
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// Stores with the device-scope cache policy (sc1), for data that the next
// kernel of the frame reads.  On the 1B and 39M frames they beat both the
// default and the non-temporal policy.  No global-store builtin takes the
// policy bits, so they go through a raw buffer resource (base = a
// wave-uniform pointer, byte offsets per lane), which the compiler schedules
// and tracks like any other store.  Callers keep a region below 2^31 bytes
// (sc1_ok) and otherwise store as before.
constexpr int CPOL_SC1 = 16;             // cache-policy operand: sc1
constexpr int BUF_WORD3 = 0x00020000;    // raw 32-bit buffer, no swizzle
__device__ __forceinline__ bool sc1_ok(long bytes) { return bytes > 0 && bytes < (1L << 31); }
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sc1_rsrc(const void* base, long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, BUF_WORD3);
}
__device__ __forceinline__ void store_sc1(__amdgpu_buffer_rsrc_t r, long off, float4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, (int)off, 0, CPOL_SC1);
}
__device__ __forceinline__ void store_sc1(__amdgpu_buffer_rsrc_t r, long off, half8_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, (int)off, 0, CPOL_SC1);
}
__device__ __forceinline__ void store_sc1(__amdgpu_buffer_rsrc_t r, long off, half4_t v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), r, (int)off, 0, CPOL_SC1);
}
// The matching device-scope load: it observes every device-scope store that
// has completed, on any CU.
__device__ __forceinline__ float4_t load_sc1_f4(__amdgpu_buffer_rsrc_t r, long off) {
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, CPOL_SC1));
}

// LDS-DMA destination pointers, explicit memory waits and the raw barrier.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt vmcnt(N) lgkmcnt(0): at most N vector-memory operations of this
// wave outstanding (they complete in issue order), no LDS operation.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | (((N >> 4) & 0x3) << 14));
}

// s_barrier without __syncthreads' release fence (which would drain vmcnt to
// zero on gfx9 and serialise prefetches that are still in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// Wave64 reductions.  Lanes 0..63 of a CDNA wave form 4 DPP rows of 16.
// Inside a row: xor-1 and xor-2 exchanges (quad_perm), then the half-row and
// row mirrors; every lane then holds its row's sum, bit-identical across the
// row (each step adds the same two operands, only commuted).  The four row
// sums are combined with readlane in a fixed order, so the result is
// deterministic and identical in every lane.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

constexpr int DPP_QUAD_1032 = 0xB1;   // quad_perm [1,0,3,2]  (xor 1)
constexpr int DPP_QUAD_2301 = 0x4E;   // quad_perm [2,3,0,1]  (xor 2)
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<DPP_QUAD_1032>(v);
  v += dpp_mov<DPP_QUAD_2301>(v);
  v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
  v += dpp_mov<DPP_ROW_MIRROR>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_mov<DPP_QUAD_1032>(v));
  v = fmaxf(v, dpp_mov<DPP_QUAD_2301>(v));
  v = fmaxf(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_mov<DPP_ROW_MIRROR>(v));
  return v;
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  float r0 = readlane_f32(v, 0), r1 = readlane_f32(v, 16);
  float r2 = readlane_f32(v, 32), r3 = readlane_f32(v, 48);
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  float r0 = readlane_f32(v, 0), r1 = readlane_f32(v, 16);
  float r2 = readlane_f32(v, 32), r3 = readlane_f32(v, 48);
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// ---------------------------------------------------------------------------
// image2d texel read with a zero border (OpenCL CLK_ADDRESS_CLAMP).
// An image param has A rows of B texels; (y, x) is a texel coordinate.
//   fl = y*B + x, fc = clamp(fl, 0, A*B-1), valid = 0<=x<B && 0<=y<A,
//   value = valid ? texel[fc] : 0.
// The load is always issued at an in-bounds address and masked afterwards.
// Reference: run_pinned2.py:56-84 (address + predicate), 355-374 (masked load).
// ---------------------------------------------------------------------------
template <typename TexelT>
__device__ __forceinline__ TexelT img_texel_zb(const TexelT* __restrict__ img, int A, int B, int y, int x) {
  int fl = y * B + x;
  int fc = min(max(fl, 0), A * B - 1);
  bool valid = (x >= 0) & (x < B) & (y >= 0) & (y < A);
  TexelT v = img[fc];
  return valid ? v : TexelT{};
}

__device__ __forceinline__ float gelu_tanh(float x) {
  const float c = 0.7978845608028654f;   // sqrt(2/pi)
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

// Same tanh-form GELU in its sigmoid form, 0.5 x (1 + tanh(u)) = x / (1 + e^{-2u}),
// with e^{-2u} = 2^(x (c0 + c1 x^2)), c0 = -2 sqrt(2/pi) log2(e), c1 = 0.044715 c0,
// on the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32): four VALU
// operations and two transcendentals per element (the GEMM epilogue runs it
// on every output, so the count sets the epilogue's time).  Large |x| saturate
// to x and -0 through inf/0 of the exp2.  The relative error is ~1e-7, far
// below the f16 rounding of the GEMM epilogue that consumes it.
__device__ __forceinline__ float gelu_fast(float x) {
  constexpr float c0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
  constexpr float c1 = 0.044715f * c0;
  const float z = x * __builtin_fmaf(c1, x * x, c0);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

inline int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

}  // namespace ck
