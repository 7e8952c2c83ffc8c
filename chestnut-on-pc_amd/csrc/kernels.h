// Host-side launchers for every device kernel of the frame.  All launchers
// validate shapes/alignment on the host before launching (a bad shape is an
// ck::Error, never an out-of-bounds access) and enqueue on the given stream.
#pragma once

#include "common.h"

namespace ck {

// ---- GEMV (serial reduce r_32_32_3_12288_32 analogue) ----------------------
// y[r] = act(sum_k W[r*ldw + k] * x[k] + bias[r]),  r < rows, k < K.
// W f16 row-major, x f32, y f32.  K % 8 == 0, ldw % 8 == 0, K <= 16384,
// W and x 16-byte aligned.  act: 0 none, 1 gelu(tanh).  rows_per_wg: 0 = auto.
enum GemvAct { GEMV_NONE = 0, GEMV_GELU = 1 };
// stream: load W non-temporal (the weights pass once; for a model whose
// weights fit the Infinity Cache the default policy keeps them there).
void launch_gemv(const half_t* W, const float* x, const float* bias, float* y, int rows, int K,
                 int ldw, int act, int rows_per_wg, hipStream_t s, bool stream = true);
// Two independent GEMVs (ldw = K, no activation) in one launch.
void launch_gemv2(const half_t* W0, const float* x0, const float* b0, float* y0, int rows0, int K0, const half_t* W1,
                  const float* x1, const float* b1, float* y1, int rows1, int K1, hipStream_t s, bool stream = true);
// y = W . h + bias with h the GRU update of gi, gh (gates r, z, n; biases
// included) and h_prev, computed inside the GEMV; h is also stored to h_out
// (and h_out2 when non-null).  W is [rows][H].
void launch_gemv_gru(const half_t* W, const float* bias, float* y, int rows, const float* gi, const float* gh,
                     const float* h_prev, float* h_out, float* h_out2, int H, hipStream_t s, bool stream = true);

// ---- MFMA GEMM (WMMA attention/projection GEMM analogue) -------------------
enum Epi {
  EPI_F32 = 0,            // C32 = acc (+ bias)
  EPI_F16_BIAS = 1,       // C16 = f16(acc + bias)
  EPI_F16_BIAS_RELU = 2,  // C16 = f16(relu(acc + bias))
  EPI_F16_BIAS_GELU = 3,  // C16 = f16(gelu(acc + bias))
  EPI_F32_RESID = 4,      // C32 += acc (+ bias)
  EPI_QKV = 5,            // f16(acc + bias): n < qk_cols -> C16[m][n], else vt[n-qk_cols][m]
  EPI_PARTIALS = 6,       // raw f32 acc of split s -> ws[s][M][N] (no bias, no reduce); a
                          // consumer (the residual-add LayerNorm) sums the splits
  EPI_EMBED = 8,          // C32 = acc + bias + pos16[m][n] + ctx[n] (the token embedding:
                          // position table and the per-frame context vector folded in)
  EPI_QKV_FRAG = 7,       // f16(acc + bias) of a [T][3d] QKV product, written in the MFMA
                          // fragment order the attention kernel loads (see gemm.hip):
                          // Q, K -> C, V -> vt.  Needs head_dim, M % 32 == 0, split 1.
};

// y = W . x + bias (W f16 [rows][K], ldw = K, x f32 [K], no activation) run by
// extra workgroups of another launch (GemmDesc::rider); rows = 0: none.
struct GemvRider {
  const half_t* W = nullptr;
  const float* x = nullptr;
  const float* bias = nullptr;
  float* y = nullptr;
  int rows = 0, K = 0;
  bool stream = true;   // non-temporal weight loads (launch_gemv's `stream`)
};

struct GemmDesc {
  const half_t* A = nullptr;   // [M][K] row-major, lda
  const half_t* B = nullptr;   // [N][K] row-major (b_kn=false) or [K][N] (b_kn=true), ldb
  void* C = nullptr;           // [M][N] row-major, ldc (f32 or f16 per epi)
  const float* bias = nullptr; // [N] or null
  long lda = 0, ldb = 0, ldc = 0;
  int M = 0, N = 0, K = 0;
  bool b_kn = false;
  int epi = EPI_F32;
  int split = 0;               // split-K factor; 0 = auto
  float* ws = nullptr;         // split-K partials: split * batch * M * N floats
  size_t ws_floats = 0;
  int batch = 1;
  long sA = 0, sB = 0, sC = 0, sBias = 0;   // per-batch element strides
  half_t* vt = nullptr;        // EPI_QKV transposed V output
  int qk_cols = 0;
  long vt_ld = 0;
  int tile = 0;                // 0 auto; else 1:128x128 2:128x64 3:64x128 4:64x64
  int head_dim = 0;            // EPI_QKV_FRAG only
  const half_t* pos = nullptr; // EPI_EMBED: f16 [M][N] position table (row stride ldc)
  const float* ctx = nullptr;  // EPI_EMBED: f32 [N] added to every row
  // Implicit 3x3 stride-2 pad-1 convolution (conv_c > 0): A is the input
  // activation f16 [batch][conv_h][conv_w][conv_c] (sA per batch image), row m
  // of the virtual patch matrix is output pixel m (M = Ho*Wo), column k =
  // tap*conv_c + channel (K = round_up(9*conv_c, 64)); border taps and the K
  // padding read the 16 zero bytes at zero16.  conv_c: a power of two >= 8.
  int conv_c = 0, conv_h = 0, conv_w = 0;
  const half_t* zero16 = nullptr;
  // Store the f16 result transposed, C[b*sC + n*ldc + m] (the split-K
  // reduce of EPI_F16_BIAS_RELU on tiles 1-8 only; requires split > 1).
  int c_nm = 0;
  // A GEMV run by extra workgroups of this GEMM's split-K reduce launch
  // (implicit conv with split > 1 only): an independent small product that
  // then costs no launch of its own.
  GemvRider rider;
};
// Resolves auto tile/split (writes them back) and returns the workspace the
// launch needs, in floats.
size_t gemm_plan(GemmDesc& d);
void launch_gemm(GemmDesc d, hipStream_t s);

// ---- attention ---------------------------------------------------------------
// Row layout (frag = false): qk f16 [T][2d] (q | k, head h at columns h*hd),
// vt f16 [d][T] (V transposed).  Fragment layout (frag = true): qk and vt as
// written by the EPI_QKV_FRAG GEMM epilogue.  out f16 [T][d].
// Non-causal softmax(q k^T * scale) v per head.
void launch_attention(const half_t* qk, const half_t* vt, half_t* out, int T, int n_heads, int head_dim, bool frag,
                      hipStream_t s);
// Attention (fragment layout) with the output projection in the same launch:
// opart + h*T*d = O_h W_o[:, h*hd:(h+1)*hd]^T, f32 [T][d], one plane per head
// (the O-projection's partials over K split by heads, summed by the next
// LayerNorm); wo f16 [d][d].  attention_oproj_tiles returns the output tiles
// per wave for a shape (0: not supported, use launch_attention + a GEMM).
int attention_oproj_tiles(int T, int n_heads, int head_dim);
void launch_attention_oproj(const half_t* qk, const half_t* vt, const half_t* wo, float* opart, int T, int n_heads,
                            int head_dim, hipStream_t s);

// ---- normalisation / small elementwise ---------------------------------------
void launch_layernorm(const float* x, const float* g, const float* b, void* out, bool out_f16, int rows,
                      int d, float eps, hipStream_t s);
// x += ((ws[0] + ws[1]) + ... + ws[nsplit-1]) + rbias (the split-K partials of
// the GEMM that produced x's update; ws[k] at ws + k*split_stride), then LN.
void launch_add_layernorm(float* x, const float* ws, int nsplit, long split_stride, const float* rbias, const float* g,
                          const float* b, void* out, bool out_f16, int rows, int d, float eps, hipStream_t s);
// out[n] = mean over rows of x[r][n] (d % 32 == 0), deterministic.
void launch_colmean(const float* x, float* out, int rows, int d, hipStream_t s);
void launch_fill_u32(void* p, unsigned v, size_t n_words, hipStream_t s);

// ---- output decode (parse_model_outputs.py Parser on device) -----------------
enum DecodeKind { DEC_RAW = 0, DEC_MDN = 1, DEC_SIGMOID = 2, DEC_SOFTMAX = 3, DEC_MHP = 4 };
struct DecodeHead {
  int kind;
  int in_off, len;   // raw slice of the output vector
  int out_off;       // start in the decoded vector
  int n;             // MDN / MHP: values per mu (and per std)
  int width;         // SOFTMAX group width
  int in_N, out_N;   // MHP hypotheses / selections (in_N <= 8, out_N <= 8)
};
// One workgroup per head; heads_dev is a device copy of the table.  With a
// counter, one more workgroup does the end-of-frame tick in the same launch:
// counter + 1 and h -> packed_feat (the prev_feat slot of the next frame).
void launch_decode(const float* raw, float* decoded, const DecodeHead* heads_dev, int n_heads, hipStream_t s,
                   unsigned* counter = nullptr, const float* h = nullptr, float* packed_feat = nullptr, int H = 0);

// ---- NV12 perspective warp -> `warped` (compile_modeld.py:53-118, 181-193) ----
// frame, big_frame: NV12 (Y plane of y_height rows, then the interleaved UV
// plane), rows of `stride` bytes, frame_bytes each; tfm, big_tfm: device f32
// [3][3] inverse transforms; out u8 [2][6][model_h/2][model_w/2].
// division: 0 src_x / src_w (correctly rounded quotient), 1 src_x * (1 / src_w)
// (correctly rounded reciprocal, then the product).
void launch_warp_nv12(const uint8_t* frame, const uint8_t* big_frame, size_t frame_bytes, const float* tfm,
                      const float* big_tfm, int cam_w, int cam_h, int stride, int y_height, int model_w, int model_h,
                      int division, uint8_t* out, hipStream_t s);

// ---- frame inputs, packing, image2d ------------------------------------------
struct QueueDims {
  int img_h, img_w;          // 128, 256
  int fs;                    // frame skip (4)
  int img_slots;             // fs*(n_frames-1)+1 (5)
  int feat_len, feat_hist;   // 512, 24
  int desire_len, desire_hist;  // 8, 25
};
// One `run_policy` input stage on device ring buffers (see pack.hip).
void launch_policy_inputs(const QueueDims& q, const uint8_t* warped, const float* packed, const unsigned* counter,
                          uint8_t* img_ring, float* feat_ring, float* desire_ring, uint8_t* img_out,
                          float* feat_out, float* ctx_tail, hipStream_t s);
void launch_yuv_to_channels(const uint8_t* Y, const uint8_t* U, const uint8_t* V, int H, int W, uint8_t* out,
                            hipStream_t s);
void launch_i420_to_channels(const uint8_t* frame, int H, int W, uint8_t* out, hipStream_t s);
// Zero-border gather: img has A rows of B texels of `lanes` elements of
// `elem_bytes` bytes; yx int32 [n][2]; out [n][lanes].
void launch_img_gather(const void* img, int A, int B, int lanes, int elem_bytes, const int* yx, int n, void* out,
                       hipStream_t s);
// Conv stem im2col (zero-border reads).  Layer 1 reads normalised uint8
// planes [batch][C][H][W]; later layers read f16 [batch][H][W][C] texels.
void launch_im2col_u8(const uint8_t* img, int batch, int C, int H, int W, half_t* patches, int Kp, hipStream_t s);
// The frame's first launch: launch_policy_inputs, the temporal GEMV
// y = act(W . features + bias) (W [rows][feat_hist*feat_len], the features
// read from the feature ring as launch_policy_inputs samples them) and
// launch_im2col_u8 of the sampled image (read from the image ring and
// `warped`), in one launch.  `slots` = resident workgroups of the launch on
// the device (frame_head_slots, queried once outside any graph capture; 0 =
// query now): the im2col is folded onto the slots the others leave free.
int frame_head_slots(int K, bool stream);
void launch_frame_head(const QueueDims& q, const uint8_t* warped, const float* packed, const unsigned* counter,
                       uint8_t* img_ring, float* feat_ring, float* desire_ring, uint8_t* img_out, float* feat_out,
                       float* ctx_tail, const half_t* Wt, const float* bias, float* y, int rows, int act, bool stream,
                       half_t* patches, int Kp, int slots, hipStream_t s);
void launch_im2col_f16(const half_t* act, int batch, int C, int H, int W, half_t* patches, int Kp, hipStream_t s);
void launch_tokens(const half_t* stem_out, int n_spatial, int C5, half_t* F, hipStream_t s);

// ---- dependent-launch cost (chain.hip) ---------------------------------------
// us per launch of `reps` repetitions of a chain of n dependent launches of a
// near-empty kernel on `workgroups` workgroups: mode 0 plain launches, mode 1
// the chain captured once as a graph and replayed.  Synchronises s.
float time_launch_chain(int n, int workgroups, int mode, int reps, hipStream_t s);
// us per launch of the 128x128-tile GEMM operand stream without arithmetic
// (mode 0: LDS-DMA ring, 4 waves; 1: the same with 8 waves; 2: register
// loads), operands rotating over `copies` copies (stream.hip).
float time_operand_stream(int M, int N, int K, int mode, int copies, int reps, hipStream_t s);

// ---- content hash of device tensors (hash.hip) --------------------------------
constexpr int HASH_SPAN_BYTES = 64 << 10;
struct HashSpan {
  const uint8_t* p;   // tensor base
  long off;           // span start, bytes (a multiple of 16)
  int n;              // span length, bytes (<= HASH_SPAN_BYTES)
  int tensor;         // index of the tensor the span belongs to (host bookkeeping)
};
__host__ __device__ uint64_t hash_mix(uint64_t z);
// partial[i] = the sum over span i's chunks; a tensor's hash is hash_mix(n)
// plus the sum of its spans' partials (mod 2^64).
void launch_state_hash(const HashSpan* spans, int n_spans, unsigned long long* partial, hipStream_t s);

// ---- KATs --------------------------------------------------------------------
// RDNA4 wave32 WMMA fragments (u16 [32][8] A, B; f32 [32][8] C) -> D fragment,
// computed on gfx950 MFMA.  n_tiles independent WMMAs.
void launch_wmma_rdna4(const uint16_t* fa, const uint16_t* fb, const float* fc, float* fd, int n_tiles,
                       hipStream_t s);
// One MFMA on plain row-major operands: variant 0 = 16x16x32 f16, 1 = 32x32x16 f16.
// A [M][K], B [K][N] (u16 f16 bits), D f32 [M][N].
void launch_mfma_kat(int variant, const uint16_t* A, const uint16_t* B, float* D, hipStream_t s);

}  // namespace ck
