/*
 * chestnut.h -- C ABI of the MI355X (gfx950) per-frame driving-model engine.
 *
 * The reference exposes its hot path as a Python namespace obtained by
 * exec-ing run_pinned2.py up to '# --- smoke run' (run_pinned2.py:1574,
 * video_check.py:18-19): run_frame, out_slices, make_warped, queues, PACKED.
 * Its device work goes through the CUDA driver API via tinygrad's ctypes
 * bindings.  This header is the native boundary that replaces both: plain
 * pointers and sizes, no framework types.  A ctypes binding of it (the
 * package's chestnut/_lib.py) restores the reference's Python surface.
 *
 * Conventions
 *  - Every function returns 0 on success and nonzero on failure; the failure
 *    message is ck_last_error() (thread-local).  The Python layer raises
 *    RuntimeError with it, as the reference's `check` does on CUDA status
 *    codes (run_pinned2.py:1317-1320, 1440).
 *  - `stream` arguments are hipStream_t passed as void* (NULL = null stream).
 *  - Device-pointer entry points validate shapes and alignment on the host
 *    and return an error instead of launching anything out of bounds.
 *  - An engine handle owns one HIP stream; it is not reentrant (one caller
 *    thread at a time), like the reference's module globals
 *    (run_pinned2.py:1424-1431).
 */
#ifndef CHESTNUT_H
#define CHESTNUT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ck_engine ck_engine;

/* Thread-local message of the last failure ("" if none).
 * Replaces: RuntimeError raised by `check` (run_pinned2.py:1317-1320). */
const char* ck_last_error(void);

/* Library version (major, minor). */
int ck_version(int* major, int* minor);

/* ------------------------------------------------------------------------ */
/* Engine: model, queues, frame plan, graph                                  */
/* ------------------------------------------------------------------------ */

/* Build an engine for a model spec (flat JSON, see chestnut/spec.py):
 * allocates parameters, queue rings, activations, resolves the frame plan.
 * Replaces: pickle load + reprepare + graph flatten + queue allocation
 * (run_pinned2.py:1346-1389). */
int ck_create(const char* spec_json, ck_engine** out);
int ck_destroy(ck_engine* e);

/* Parameter table (same order as chestnut/spec.py param_table).
 * dtype: 0 = f32, 1 = f16.  nbytes = logical (unpadded) size.
 * Replaces: the weights carried inside the pickle (run_pinned2.py:1349). */
int ck_param_count(ck_engine* e, int* n);
int ck_param_info(ck_engine* e, int i, char* name, size_t name_len, size_t* nbytes, int* dtype);
int ck_upload_param(ck_engine* e, const char* name, const void* host, size_t nbytes);

/* Output vector size and the name -> [start, stop) map as JSON, e.g.
 * {"plan":[0,990],...,"hidden_state":[1673,2185]}.
 * Replaces: out_slices = meta['output_slices'] (run_pinned2.py:1353-1354). */
int ck_output_size(ck_engine* e, int* n);
int ck_output_slices(ck_engine* e, char* buf, size_t len);

/* Parsed outputs.  Every frame ends with the Parser's decode on device
 * (MDN mu / safe_exp std, sigmoid, grouped softmax, multi-hypothesis
 * selection, by head name); the f32 result is the state tensor "decoded"
 * (read it with ck_read_tensor).  This returns its length and its layout as
 * JSON: {head: {"kind": "mdn"|"sigmoid"|"softmax"|"mhp"|"raw", ranges...}}.
 * Replaces: Parser.parse_outputs on the sliced output vector
 * (parse_model_outputs.py:95-120; modeld.py:161-162, 195). */
int ck_decoded_layout(ck_engine* e, int* n, char* buf, size_t len);

/* One policy frame.  warped: uint8 [2][6][img_h][img_w] host array;
 * packed: f32 [desire 8 | traffic_convention 2 | action_t 2 | prev_feat 512];
 * out: f32 [ck_output_size].  The first call (graph mode) captures the plan
 * into a hipGraph; every call is H2D staging + one graph launch + D2H.
 * Replaces: run_frame(warped_np, packed) (run_pinned2.py:1462-1565). */
int ck_run_frame(ck_engine* e, const uint8_t* warped, const float* packed, float* out);

/* The openpilot flow of one step: two NV12 camera frames (frame_bytes each,
 * the geometry of the spec's "camera" object) and their f32 [3][3] inverse
 * transforms are warped on device into `warped` (see ck_warp_nv12), then the
 * frame runs as in ck_run_frame.  Host pointers.
 * Replaces: warp(tfm, big_tfm, frame, big_frame) followed by run_policy
 * (compile_modeld.py:181-221; modeld's per-frame call). */
int ck_run_frame_nv12(ck_engine* e, const uint8_t* frame, const uint8_t* big_frame, size_t frame_bytes,
                      const float* tfm, const float* big_tfm, const float* packed, float* out);

/* 1 = replay the plan as one hipGraph launch per frame (default),
 * 0 = launch the plan kernel by kernel.
 * Replaces: REPLAY=1 / REPLAY=0 (run_pinned2.py:1391-1403, 1567-1571). */
int ck_set_graph(ck_engine* e, int on);
int ck_graph_nodes(ck_engine* e, size_t* n);

/* Zero the queues and the frame counter (fresh input queues).
 * Replaces: make_input_queues (compile_modeld.py:149-163, run_pinned2.py:1379-1386). */
int ck_reset(ck_engine* e);

/* Device-resident frame: launch the frame on the engine's own input tensors
 * ("warped", "packed") without host copies and without synchronising.  The
 * frame ends by writing its hidden state into packed's prev_feat slot, so
 * back-to-back launches are the recurrent frame loop of
 * run_pinned2.py:1576-1587 with the host round trip removed. */
int ck_frame_launch(ck_engine* e);
int ck_synchronize(ck_engine* e);
int ck_stream(ck_engine* e, void** stream);

/* Resolved plan: number of launches and, per launch, its plan name, kernel
 * family and algorithmic flops / HBM bytes.
 * Replaces: the recorded _plan list (run_pinned2.py:1466-1475). */
int ck_plan_size(ck_engine* e, int* n);
int ck_plan_entry(ck_engine* e, int i, char* name, size_t name_len, char* kernel, size_t kernel_len, double* flops,
                  double* bytes);

/* Run one eager frame with an event pair around every launch and a
 * synchronise after each; ms[i] = launch i's time.  n >= plan size.
 * Replaces: KSYNC=1 (run_pinned2.py:1513-1557). */
int ck_kernel_times(ck_engine* e, float* ms, int n);

/* Launch plan entries [first, last) eagerly and synchronise.
 * Replaces: the per-launch bisect of research/xcheck.py:65-124 (XINJECT). */
int ck_run_range(ck_engine* e, int first, int last);

/* Launch plan entries idx[0..n) in order, `reps` times over, between two HIP
 * events recorded on the engine's stream; *ms = elapsed time of all
 * n * reps launches.  Used to time one kernel family live (e.g. every
 * layer's MLP-up GEMM, so each launch streams its own weights).
 * Replaces: the per-kernel bench loop of bench_r62.py:25-37. */
int ck_time_launches(ck_engine* e, const int* idx, int n, int reps, float* ms);

/* Run `frames` whole eager frames back to back (no synchronisation between
 * launches, the frame's state advancing as usual) and time the kernels of
 * plan entries idx[0..n) by their own dispatch start and end timestamps:
 * per_entry_ms[k] = entry idx[k]'s kernel time per frame (may be NULL),
 * *mean_ms = the mean over the n entries (may be NULL).  The in-frame
 * duration a kernel trace reports, measured without a profiler.
 * Replaces: KTIME=1, per-kernel GPU time over a run (run_pinned2.py:1307-1329). */
int ck_time_in_frames(ck_engine* e, const int* idx, int n, int frames, float* per_entry_ms, float* mean_ms);

/* Named device tensors (parameters, inputs, queue rings, activations):
 * device pointer + logical size, and synchronous host copies.
 * Replaces: KDUMP pre-state dumps (run_pinned2.py:1533-1545) and the
 * probes' cuMemcpyDtoH captures (r62_probe.py:28-37). */
int ck_tensor(ck_engine* e, const char* name, void** dptr, size_t* nbytes);
/* Frame state: the non-parameter tensors (inputs, rings, activations, the
 * split-K workspace "ws"), in allocation order.  dtype as ck_param_info plus
 * 2 = u8, 3 = u32.  A probe snapshots all of them around one plan entry.
 * Replaces: the probes' per-argument span discovery (r62_probe.py:31-35). */
int ck_state_count(ck_engine* e, int* n);
int ck_state_info(ck_engine* e, int i, char* name, size_t name_len, size_t* nbytes, int* dtype);
/* A 64-bit content hash of every state tensor (ck_state_info order, whole
 * tensor, computed on the device after the work queued on the engine
 * stream; synchronises).  Taken before each launch of an eager frame it is
 * the launch's pre-state fingerprint; two runs' fingerprints name the first
 * launch after which they diverge, and which tensors differ.  n >= the
 * state count.
 * Replaces: KSYNC's md5 of each launch's argument pre-state
 * (run_pinned2.py:1519-1542) and research/xcheck.py's per-argument hashes
 * (research/xcheck.py:65-124). */
int ck_state_hashes(ck_engine* e, uint64_t* out, int n);

/* The cost of a dependent launch: `reps` repetitions of a chain of n_launches
 * launches of a near-empty kernel over `workgroups` workgroups, each ordered
 * after the previous one on `stream`; mode 0 = plain launches, 1 = the chain
 * captured once as a graph and replayed (one graph launch per repetition).
 * *us_per_launch = elapsed time / (n_launches * reps), HIP events on stream
 * (a null stream: a stream the call creates and destroys, since the null
 * stream cannot be captured).
 * Replaces: the reference's launch-cost measurements of its frame plan,
 * ~0.5 ms per frame outside a CUDA graph, ~1.6 us per launch inside
 * (README.md:20-26, 73; NOTES.md:48-50). */
int ck_time_launch_chain(int n_launches, int workgroups, int mode, int reps, float* us_per_launch, void* stream);

/* The operand stream of a block GEMM (C = A B^T, A [M][K], B [N][K]) with its
 * arithmetic taken out: the 128x128-tile grid, XCD-grouped tile order,
 * 64-wide K-steps and per-step waits of the LDS-DMA GEMM, no MFMA, no
 * fragment reads, no epilogue.  mode 0: LDS-DMA into a 4-stage ring, 4 waves;
 * 1: the same with 8 waves; 2: 16-byte loads into registers, no LDS; 3: mode 0
 * on 128x96 tiles (the QKV GEMM's).  A and B rotate over `copies` copies
 * (enough of them and B streams from HBM as the weights of a frame do);
 * *us_per_launch: HIP events over `reps` launches after `reps` untimed ones.
 * M a multiple of 128, N of the tile width (128, or 96 in mode 3), K of 64.
 * Replaces: the reference's per-kernel bench loop (bench_r62.py:25-37)
 * applied to the GEMM's loads alone. */
int ck_time_operand_stream(int M, int N, int K, int mode, int copies, int reps, float* us_per_launch, void* stream);
int ck_read_tensor(ck_engine* e, const char* name, void* host, size_t nbytes);
int ck_write_tensor(ck_engine* e, const char* name, const void* host, size_t nbytes);

/* ------------------------------------------------------------------------ */
/* Per-kernel entry points (device pointers) for the probe / bench harness  */
/* ------------------------------------------------------------------------ */

/* y[r] = act(sum_k W[r*ldw+k] x[k] + bias[r]); W f16, x/y/bias f32; bias may
 * be NULL; act 0 = none, 1 = gelu(tanh).  K % 8 == 0, K <= 16384, ldw % 8 == 0,
 * W and x 16-byte aligned.  rows_per_wg 0 = automatic.
 * Replaces: launch of r_32_32_3_12288_32 (bench_alu.py:13-29; its
 * warp-split form run_pinned2.py:989-1066). */
int ck_gemv(const void* W, const float* x, const float* bias, float* y, int rows, int K, int ldw, int act,
            int rows_per_wg, void* stream);

/* C f32 [M][N] = A f16 [M][K] (lda) * B, B f16 either [K][N] (b_kn = 1, ldb)
 * or [N][K] (b_kn = 0, ldb); optional bias f32 [N].  K % 64 == 0.
 * tile: 0 auto, 1 128x128, 2 128x64, 3 64x128, 4 64x64 (5-8: the same tiles
 * with one K-group; 9: 256x128 with 8 waves; 11, 13: the register-staged
 * kernel; 10, 128x96, serves only the frame plan's QKV epilogue; 15: 32x64
 * with two waves, B as [N][K]); split_k: 0 auto.
 * workspace: split_k * M * N floats when split_k > 1, plus, for a [K][N] B
 * on tiles 1-8, N * K halves for B transposed to [N][K] (query with
 * ck_gemm_workspace, which also resolves auto tile/split).
 * split_k = 2 on tile 2 ([K][N] B) or on tiles 2-4 ([N][K] B, K per split a
 * multiple of 128) finishes inside the GEMM launch (no reduce launch): the
 * result is bit for bit the reduce's.  It counts finished workgroups in a
 * static per-device array with a slot per stream (16 streams per device;
 * later streams get the reduce launch), so such calls may run at the same
 * time on different streams; a graph captured with such a call keeps its
 * capturing stream's slot and must not run while that stream runs one.
 * Replaces: launch of the WMMA GEMM kernels r_6_2 / r_2_24 / r_12_32_4 /
 * r_48_32_4 (bench_r62.py:13-29, bench_r12.py, bench_r48.py). */
int ck_gemm_workspace(int M, int N, int K, int b_kn, int* tile, int* split_k, size_t* ws_bytes);
int ck_gemm(const void* A, const void* B, float* C, const float* bias, int M, int N, int K, long lda, long ldb,
            long ldc, int b_kn, int tile, int split_k, void* workspace, size_t ws_bytes, void* stream);

/* ck_gemm without the workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * The split-K partials (and a transposed [K][N] B where the tile needs one)
 * go to a static 32 MiB device array per GPU, held until the process ends;
 * the call allocates nothing.  A GEMM whose workspace (ck_gemm_workspace)
 * exceeds 32 MiB is rejected with an error.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams, other
 * threads) race.  The device of `stream` must be the current device. */
int ck_gemm_noalloc(const void* A, const void* B, float* C, const float* bias, int M, int N, int K, long lda,
                    long ldb, long ldc, int b_kn, int tile, int split_k, void* stream);

/* f16 GEMM with a fused epilogue, as the frame plan uses it.
 * epi: 1 f16(acc+bias), 2 f16(relu(acc+bias)), 3 f16(gelu(acc+bias)),
 *      4 C f32 += acc + bias.  B is [N][K]. */
int ck_gemm_epi(const void* A, const void* B, void* C, const float* bias, int M, int N, int K, long lda, long ldb,
                long ldc, int epi, int tile, int split_k, void* workspace, size_t ws_bytes, void* stream);

/* NV12 camera frames -> the 6-channel model input `warped`: perspective
 * warp with nearest-neighbour sampling (f32 coordinates, round half to
 * even, clipped to the edge), Y at model_w x model_h, U and V from the
 * interleaved UV plane at half resolution, packed as frames_to_tensor does.
 * frame, big_frame: device NV12 buffers of frame_bytes (Y plane: y_height
 * rows of stride bytes, then the UV plane); tfm, big_tfm: device f32 [3][3]
 * inverse transforms; out: device u8 [2][6][model_h/2][model_w/2].
 * division: how src_x / src_w is evaluated -- 0 the correctly rounded f32
 * quotient, 1 the product with the correctly rounded f32 reciprocal (the
 * reference writes the quotient, compile_modeld.py:65-66, and its engine
 * lowers f32 divisions to x * rcp(y), run_pinned2.py:622-628; the forms
 * pick different texels at a few .5 boundaries per frame).
 * Replaces: make_warp / frame_prepare_tinygrad / warp_perspective_tinygrad
 * (compile_modeld.py:53-118, 181-193). */
int ck_warp_nv12(const uint8_t* frame, const uint8_t* big_frame, size_t frame_bytes, const float* tfm,
                 const float* big_tfm, int cam_w, int cam_h, int stride, int y_height, int model_w, int model_h,
                 int division, uint8_t* out, void* stream);

/* n_tiles WMMA uops ((16,16,16), half, 'AMD', 32): per tile u16 fragA[32][8],
 * fragB[32][8], f32 fragC[32][8] -> f32 fragD[32][8], RDNA4 lane layout.
 * Replaces: _wm_emit's WMMA lowering (run_pinned2.py:119-266) and the
 * consumer probe (consumer_probe.py). */
int ck_wmma_rdna4(const uint16_t* fragA, const uint16_t* fragB, const float* fragC, float* fragD, int n_tiles,
                  void* stream);

/* One MFMA on row-major operands (variant 0: 16x16x32, A [16][32], B [32][16];
 * variant 1: 32x32x16, A [32][16], B [16][32]) -> D f32.  Layout KAT for the
 * operand maps the GEMM and attention kernels use.
 * Replaces: mma_probe.py's fragment-layout probe (mma_probe.py:10-105). */
int ck_mfma_kat(int variant, const uint16_t* A, const uint16_t* B, float* D, void* stream);

/* YUV planes uint8 [H][W] each -> uint8 [6][H/2][W/2] = Y00,Y10,Y01,Y11,U,V.
 * Replaces: rgb_to_channels' packing (video_check.py:27-32). */
int ck_pack_yuv(const uint8_t* Y, const uint8_t* U, const uint8_t* V, int H, int W, uint8_t* out, void* stream);

/* I420 frame uint8 [H*3/2][W] -> uint8 [6][H/2][W/2].
 * Replaces: frames_to_tensor (compile_modeld.py:83-92). */
int ck_frames_to_tensor(const uint8_t* frame, int H, int W, uint8_t* out, void* stream);

/* Zero-border image2d gather: img = A rows x B texels x lanes elements of
 * elem_bytes; yx = int32 [n][2] (y, x); out [n][lanes].
 * Replaces: the image branch of _addrflat + masked LOAD
 * (run_pinned2.py:56-84, 355-374); semantics of research/probe_sampler.py. */
int ck_img_gather(const void* img, int A, int B, int lanes, int elem_bytes, const int32_t* yx, int n, void* out,
                  void* stream);

/* Multi-head attention on a packed QK tensor f16 [T][2d] and V^T f16 [d][T]
 * -> f16 [T][d].  T % 64 == 0, T <= 512, head_dim 64 or 128. */
int ck_attention(const void* qk, const void* vt, void* out, int T, int n_heads, int head_dim, void* stream);

/* Row LayerNorm of x f32 [rows][d] -> f16 (out_f16 = 1) or f32. */
int ck_layernorm(const float* x, const float* g, const float* b, void* out, int out_f16, int rows, int d, float eps,
                 void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CHESTNUT_H */
