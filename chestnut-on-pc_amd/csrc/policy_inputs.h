// Policy input queues on device rings: the work of one `run_policy` input
// stage as a device function, shared by its own kernel (pack.hip) and by the
// frame-head launch (gemv.hip).
#pragma once

#include "common.h"
#include "kernels.h"

namespace ck {

__device__ __forceinline__ int wrap(long f, int n) {
  long r = f % n;
  return (int)(r < 0 ? r + n : r);
}

// ---------------------------------------------------------------------------
// Policy input queues on ring buffers.
//
// The reference shifts every queue by one entry per frame and samples it
// (shift_and_sample / sample_skip / sample_desire, compile_modeld.py:166-176,
// called from run_policy, compile_modeld.py:198-212).  Here each queue is a
// ring indexed by the device frame counter n (frames pushed so far), so no
// entry is ever moved.  After the push of frame n the reference's queue
// position j of a length-L queue holds the entry of frame n-L+1+j, which
// lives in ring slot (n-L+1+j) mod L; slots never written are still zero, as
// the reference's zero-initialised queues are.  The entry of frame n itself
// is read from the input staging, never from the slot written in this same
// launch, so no workgroup depends on another's store.
//   img:    L = 5,   sample j = 0, 4        -> frames n-4 and n
//   feat:   L = 96,  sample j = 0, 4, .., 92 -> frames n-95+4i (n only when
//           frame_skip = 1: its last sample, read from the staging)
//   desire: L = 100, group g = max over j = 4g..4g+3 (frame n in group 24)
// ---------------------------------------------------------------------------
struct PolicyArgs {
  const uint8_t* warped;   // [2][6][H][W]
  const float* packed;     // desire | tc2 | action_t2 | prev_feat
  const unsigned* counter;
  uint8_t* img_ring;       // [2][img_slots][6][H][W]
  float* feat_ring;        // [fs*feat_hist][feat_len]
  float* desire_ring;      // [fs*desire_hist][desire_len]
  uint8_t* img_out;        // [2][6*n_frames][H][W]
  float* feat_out;         // [feat_hist][feat_len]
  float* ctx_tail;         // desire_pulse [desire_hist*desire_len] | tc2 | action_t2
  int frame_units;         // 16-byte units per 6-channel frame
  int img_slots, fs, feat_len, feat_hist, desire_len, desire_hist;
  int n_img, n_feat, n_feat_push, n_des, n_des_push;   // work-range sizes
};

// Work item i of one policy-input stage (policy_inputs_threads items).
__device__ __forceinline__ void policy_inputs_at(const PolicyArgs& a, long i) {
  const long n = a.counter[0];
  if (i < a.n_img) {   // two streams x frame_units: sample frames n-4 (ring) and n (staging); push n
    const int s = (int)(i / a.frame_units), u = (int)(i % a.frame_units);
    const long fb = (long)a.frame_units * 16;
    const u32x4_t cur = reinterpret_cast<const u32x4_t*>(a.warped + s * fb)[u];
    const int old_slot = wrap(n - (a.img_slots - 1), a.img_slots);
    const int new_slot = wrap(n, a.img_slots);
    uint8_t* ring = a.img_ring + (long)s * a.img_slots * fb;
    const u32x4_t old = reinterpret_cast<const u32x4_t*>(ring + old_slot * fb)[u];
    // device-scope stores (store_sc1): the conv stem reads these next
    const __amdgpu_buffer_rsrc_t ro = sc1_rsrc(a.img_out, 4L * fb);
    const __amdgpu_buffer_rsrc_t rr = sc1_rsrc(a.img_ring, 2L * a.img_slots * fb);
    store_sc1(ro, (long)s * 2 * fb + 16L * u, __builtin_bit_cast(float4_t, old));
    store_sc1(ro, (long)s * 2 * fb + fb + 16L * u, __builtin_bit_cast(float4_t, cur));
    store_sc1(rr, ((long)s * a.img_slots + new_slot) * fb + 16L * u, __builtin_bit_cast(float4_t, cur));
    return;
  }
  i -= a.n_img;
  const int fL = a.fs * a.feat_hist;
  const float* prev_feat = a.packed + a.desire_len + 4;
  if (i < a.n_feat) {   // feat_hist x feat_len samples
    const int k = (int)(i / a.feat_len), c = (int)(i % a.feat_len);
    const long f = n - (fL - 1) + (long)a.fs * k;
    a.feat_out[i] = (f == n) ? prev_feat[c] : a.feat_ring[(long)wrap(f, fL) * a.feat_len + c];
    return;
  }
  i -= a.n_feat;
  if (i < a.n_feat_push) {
    a.feat_ring[(long)wrap(n, fL) * a.feat_len + i] = prev_feat[i];
    return;
  }
  i -= a.n_feat_push;
  const int dL = a.fs * a.desire_hist;
  if (i < a.n_des) {   // desire_hist x desire_len group maxima
    const int g = (int)(i / a.desire_len), c = (int)(i % a.desire_len);
    float m = 0.f;
    for (int t = 0; t < a.fs; ++t) {
      const int j = g * a.fs + t;
      const long f = n - (dL - 1) + j;
      const float v = (j == dL - 1) ? a.packed[c] : a.desire_ring[(long)wrap(f, dL) * a.desire_len + c];
      m = (t == 0 || v > m) ? v : m;
    }
    a.ctx_tail[i] = m;
    return;
  }
  i -= a.n_des;
  if (i < a.n_des_push) {
    a.desire_ring[(long)wrap(n, dL) * a.desire_len + i] = a.packed[i];
    return;
  }
  i -= a.n_des_push;
  if (i < 4) a.ctx_tail[a.desire_hist * a.desire_len + i] = a.packed[a.desire_len + i];   // tc2 | action_t2
}

inline PolicyArgs make_policy_args(const QueueDims& q, const uint8_t* warped, const float* packed,
                                   const unsigned* counter, uint8_t* img_ring, float* feat_ring, float* desire_ring,
                                   uint8_t* img_out, float* feat_out, float* ctx_tail) {
  const long frame_bytes = 6L * q.img_h * q.img_w;
  CK_REQUIRE(frame_bytes % 16 == 0, "policy_inputs: frame size must be a multiple of 16 bytes");
  CK_REQUIRE(q.img_slots == q.fs + 1, "policy_inputs: two sampled frames expected (fs*(2-1)+1 slots)");
  // the image copies leave through raw buffer stores addressed by 32-bit offsets
  CK_REQUIRE(4L * frame_bytes < (1L << 31) && 2L * q.img_slots * frame_bytes < (1L << 31),
             "policy_inputs: image buffers must be under 2 GiB");
  PolicyArgs a;
  a.warped = warped; a.packed = packed; a.counter = counter;
  a.img_ring = img_ring; a.feat_ring = feat_ring; a.desire_ring = desire_ring;
  a.img_out = img_out; a.feat_out = feat_out; a.ctx_tail = ctx_tail;
  a.frame_units = (int)(frame_bytes / 16);
  a.img_slots = q.img_slots; a.fs = q.fs;
  a.feat_len = q.feat_len; a.feat_hist = q.feat_hist; a.desire_len = q.desire_len; a.desire_hist = q.desire_hist;
  a.n_img = 2 * a.frame_units;
  a.n_feat = q.feat_hist * q.feat_len;
  a.n_feat_push = q.feat_len;
  a.n_des = q.desire_hist * q.desire_len;
  a.n_des_push = q.desire_len;
  return a;
}

inline long policy_inputs_threads(const PolicyArgs& a) {
  return (long)a.n_img + a.n_feat + a.n_feat_push + a.n_des + a.n_des_push + 4;
}

}  // namespace ck
