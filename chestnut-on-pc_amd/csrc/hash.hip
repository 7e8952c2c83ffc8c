// Content hash of device tensors, for launch-by-launch comparison of two runs:
// the replacement of KSYNC's md5 of each launch's argument pre-state
// (run_pinned2.py:1519-1542) and of research/xcheck.py's per-argument hashes
// (research/xcheck.py:65-124).  Those read every argument back to the host
// and hash it there; here the GPU hashes whole tensors in place and only one
// 8-byte partial per 64 KiB span crosses PCIe.
//
// The hash of a tensor of n bytes is
//   mix(n) + sum over 16-byte chunks c of  mix(lo_c ^ mix(2c)) + mix(hi_c ^ mix(2c + 1))
//          + sum over tail bytes b at byte position q of  mix(b ^ mix(q + 2^62))
// modulo 2^64, with mix the splitmix64 finaliser (Steele, Lea and Flood,
// "Fast splittable pseudorandom number generators", 2014).  Each term depends
// on its position, so moved data changes the hash, and the sum is an integer
// sum: the same in any order, so the result does not depend on how the work
// is split over workgroups.  It is a fingerprint for finding where two runs
// diverge, not a cryptographic digest.
#include "common.h"
#include "kernels.h"

namespace ck {

__host__ __device__ uint64_t hash_mix(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

namespace {

// One workgroup per span: bytes [off, off + n) of a tensor starting at p
// (p + off 16-byte aligned, n <= HASH_SPAN_BYTES).  partial[blockIdx.x] = the
// span's share of the tensor's sum.
__global__ __launch_bounds__(256) void state_hash_kernel(const HashSpan* __restrict__ spans,
                                                          unsigned long long* __restrict__ partial) {
  const HashSpan sp = spans[blockIdx.x];
  const int tid = threadIdx.x;
  const uint8_t* base = sp.p + sp.off;
  const int n16 = sp.n >> 4;
  const uint64_t c0 = (uint64_t)(sp.off >> 4);
  uint64_t acc = 0;
  for (int c = tid; c < n16; c += 256) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(base + 16L * c);
    const uint64_t lo = (uint64_t)v[0] | ((uint64_t)v[1] << 32), hi = (uint64_t)v[2] | ((uint64_t)v[3] << 32);
    const uint64_t ci = c0 + (uint64_t)c;
    acc += hash_mix(lo ^ hash_mix(2 * ci)) + hash_mix(hi ^ hash_mix(2 * ci + 1));
  }
  const int tail = sp.n & 15;
  if (tid < tail) {
    const uint64_t q = (uint64_t)(sp.off + 16L * n16 + tid);
    acc += hash_mix((uint64_t)base[16L * n16 + tid] ^ hash_mix(q + (1ull << 62)));
  }
  // workgroup sum: lanes by xor shuffles, then the 4 waves through LDS in order
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += (uint64_t)__shfl_xor((unsigned long long)acc, o, 64);
  __shared__ unsigned long long wsum[4];
  if ((tid & 63) == 0) wsum[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) partial[blockIdx.x] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

}  // namespace

void launch_state_hash(const HashSpan* spans, int n_spans, unsigned long long* partial, hipStream_t s) {
  CK_REQUIRE(spans && partial && n_spans > 0, "state_hash: bad arguments");
  CK_LAUNCH(state_hash_kernel, dim3(n_spans), dim3(256), 0, s, spans, partial);
  CK_LAUNCHED("state_hash");
}

}  // namespace ck
