// extern "C" entry points declared in include/chestnut.h.  Each one catches
// every exception, records its message in the thread-local last-error slot
// and returns 1; success returns 0.
#include <cstring>
#include <sstream>
#include <string>

#include "../../include/chestnut.h"
#include "engine.h"

namespace ck {
namespace {
thread_local std::string g_last_error;
}
void set_last_error(const std::string& msg) { g_last_error = msg; }
}  // namespace ck

using namespace ck;

#define CK_API_BEGIN try {
#define CK_API_END                                   \
  }                                                  \
  catch (const std::exception& ex) {                 \
    ck::set_last_error(ex.what());                   \
    return 1;                                        \
  }                                                  \
  catch (...) {                                      \
    ck::set_last_error("unknown native exception");  \
    return 1;                                        \
  }                                                  \
  return 0;

static hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

static void copy_str(const std::string& s, char* buf, size_t len) {
  CK_REQUIRE(buf && len > s.size(), "string buffer too small");
  std::memcpy(buf, s.c_str(), s.size() + 1);
}

extern "C" {

const char* ck_last_error(void) { return ck::g_last_error.c_str(); }

int ck_version(int* major, int* minor) {
  CK_API_BEGIN
  if (major) *major = 0;
  if (minor) *minor = 1;
  CK_API_END
}

int ck_create(const char* spec_json, ck_engine** out) {
  CK_API_BEGIN
  CK_REQUIRE(spec_json && out, "ck_create: null argument");
  *out = nullptr;
  *out = new ck_engine(spec_json);
  CK_API_END
}

int ck_destroy(ck_engine* e) {
  CK_API_BEGIN
  delete e;
  CK_API_END
}

int ck_param_count(ck_engine* e, int* n) {
  CK_API_BEGIN
  CK_REQUIRE(e && n, "null argument");
  int c = 0;
  for (auto& t : e->tensors) c += t.param ? 1 : 0;
  *n = c;
  CK_API_END
}

int ck_param_info(ck_engine* e, int i, char* name, size_t name_len, size_t* nbytes, int* dtype) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  int c = 0;
  for (auto& t : e->tensors) {
    if (!t.param) continue;
    if (c++ == i) {
      copy_str(t.name, name, name_len);
      if (nbytes) *nbytes = t.nbytes;
      if (dtype) *dtype = t.dtype;
      return 0;
    }
  }
  throw Error("ck_param_info: index out of range");
  CK_API_END
}

int ck_state_count(ck_engine* e, int* n) {
  CK_API_BEGIN
  CK_REQUIRE(e && n, "null argument");
  int c = 0;
  for (auto& t : e->tensors) c += t.param ? 0 : 1;
  *n = c;
  CK_API_END
}

int ck_state_info(ck_engine* e, int i, char* name, size_t name_len, size_t* nbytes, int* dtype) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  int c = 0;
  for (auto& t : e->tensors) {
    if (t.param) continue;
    if (c++ == i) {
      copy_str(t.name, name, name_len);
      if (nbytes) *nbytes = t.nbytes;
      if (dtype) *dtype = t.dtype;
      return 0;
    }
  }
  throw Error("ck_state_info: index out of range");
  CK_API_END
}

int ck_upload_param(ck_engine* e, const char* name, const void* host, size_t nbytes) {
  CK_API_BEGIN
  CK_REQUIRE(e && name && host, "null argument");
  CK_REQUIRE(e->tensor(name).param, std::string("not a parameter: ") + name);
  e->upload(name, host, nbytes);
  CK_API_END
}

int ck_output_size(ck_engine* e, int* n) {
  CK_API_BEGIN
  CK_REQUIRE(e && n, "null argument");
  *n = e->n_out;
  CK_API_END
}

int ck_decoded_layout(ck_engine* e, int* n, char* buf, size_t len) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  if (n) *n = e->n_decoded;
  if (buf) copy_str(e->dec_layout, buf, len);
  CK_API_END
}

int ck_output_slices(ck_engine* e, char* buf, size_t len) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  std::ostringstream os;
  os << "{";
  int off = 0;
  for (auto& o : e->sp.outputs) {
    os << "\"" << o.first << "\":[" << off << "," << off + o.second << "],";
    off += o.second;
  }
  os << "\"hidden_state\":[" << off << "," << off + e->sp.hidden << "]}";
  copy_str(os.str(), buf, len);
  CK_API_END
}

int ck_run_frame(ck_engine* e, const uint8_t* warped, const float* packed, float* out) {
  CK_API_BEGIN
  CK_REQUIRE(e && warped && packed && out, "ck_run_frame: null argument");
  e->run_frame(warped, packed, out);
  CK_API_END
}

int ck_run_frame_nv12(ck_engine* e, const uint8_t* frame, const uint8_t* big_frame, size_t frame_bytes,
                      const float* tfm, const float* big_tfm, const float* packed, float* out) {
  CK_API_BEGIN
  CK_REQUIRE(e && frame && big_frame && tfm && big_tfm && packed && out, "null argument");
  CK_REQUIRE(frame_bytes == e->nv12_bytes, "run_frame_nv12: frame_bytes " + std::to_string(frame_bytes) +
                                               " != the camera's NV12 size " + std::to_string(e->nv12_bytes));
  e->run_frame_nv12(frame, big_frame, tfm, big_tfm, packed, out);
  CK_API_END
}

int ck_set_graph(ck_engine* e, int on) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  e->use_graph = on != 0;
  CK_API_END
}

int ck_graph_nodes(ck_engine* e, size_t* n) {
  CK_API_BEGIN
  CK_REQUIRE(e && n, "null argument");
  *n = e->graph_nodes;
  CK_API_END
}

int ck_reset(ck_engine* e) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  e->reset_state();
  CK_API_END
}

int ck_frame_launch(ck_engine* e) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  e->frame_launch();
  CK_API_END
}

int ck_synchronize(ck_engine* e) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  CK_HIP(hipStreamSynchronize(e->stream));
  CK_API_END
}

int ck_stream(ck_engine* e, void** stream) {
  CK_API_BEGIN
  CK_REQUIRE(e && stream, "null argument");
  *stream = e->stream;
  CK_API_END
}

int ck_plan_size(ck_engine* e, int* n) {
  CK_API_BEGIN
  CK_REQUIRE(e && n, "null argument");
  *n = (int)e->plan.size();
  CK_API_END
}

int ck_plan_entry(ck_engine* e, int i, char* name, size_t name_len, char* kernel, size_t kernel_len, double* flops,
                  double* bytes) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  CK_REQUIRE(i >= 0 && i < (int)e->plan.size(), "ck_plan_entry: index out of range");
  const Launch& l = e->plan[i];
  if (name) copy_str(l.name, name, name_len);
  if (kernel) copy_str(l.kernel, kernel, kernel_len);
  if (flops) *flops = l.flops;
  if (bytes) *bytes = l.bytes;
  CK_API_END
}

int ck_kernel_times(ck_engine* e, float* ms, int n) {
  CK_API_BEGIN
  CK_REQUIRE(e && ms, "null argument");
  e->kernel_times(ms, n);
  CK_API_END
}

int ck_time_launch_chain(int n_launches, int workgroups, int mode, int reps, float* us_per_launch, void* stream) {
  CK_API_BEGIN
  CK_REQUIRE(us_per_launch, "null argument");
  *us_per_launch = time_launch_chain(n_launches, workgroups, mode, reps, as_stream(stream));
  CK_API_END
}

int ck_time_operand_stream(int M, int N, int K, int mode, int copies, int reps, float* us_per_launch, void* stream) {
  CK_API_BEGIN
  CK_REQUIRE(us_per_launch, "null argument");
  *us_per_launch = time_operand_stream(M, N, K, mode, copies, reps, as_stream(stream));
  CK_API_END
}

int ck_state_hashes(ck_engine* e, uint64_t* out, int n) {
  CK_API_BEGIN
  CK_REQUIRE(e && out, "null argument");
  e->state_hashes(out, n);
  CK_API_END
}

int ck_run_range(ck_engine* e, int first, int last) {
  CK_API_BEGIN
  CK_REQUIRE(e, "null engine");
  e->run_range(first, last);
  CK_API_END
}

int ck_time_launches(ck_engine* e, const int* idx, int n, int reps, float* ms) {
  CK_API_BEGIN
  CK_REQUIRE(e && idx && ms && n > 0 && reps > 0, "ck_time_launches: bad arguments");
  *ms = e->time_launches(idx, n, reps);
  CK_API_END
}

int ck_time_in_frames(ck_engine* e, const int* idx, int n, int frames, float* per_entry_ms, float* mean_ms) {
  CK_API_BEGIN
  CK_REQUIRE(e && idx && n > 0 && frames > 0, "ck_time_in_frames: bad arguments");
  const float m = e->time_in_frames(idx, n, frames, per_entry_ms);
  if (mean_ms) *mean_ms = m;
  CK_API_END
}

int ck_tensor(ck_engine* e, const char* name, void** dptr, size_t* nbytes) {
  CK_API_BEGIN
  CK_REQUIRE(e && name, "null argument");
  Tensor& t = e->tensor(name);
  if (dptr) *dptr = t.ptr;
  if (nbytes) *nbytes = t.nbytes;
  CK_API_END
}

int ck_read_tensor(ck_engine* e, const char* name, void* host, size_t nbytes) {
  CK_API_BEGIN
  CK_REQUIRE(e && name && host, "null argument");
  Tensor& t = e->tensor(name);
  CK_REQUIRE(t.ld == t.cols, std::string("ck_read_tensor: padded tensor ") + name);
  CK_REQUIRE(nbytes <= t.nbytes, std::string("ck_read_tensor: size exceeds ") + name);
  CK_HIP(hipStreamSynchronize(e->stream));
  CK_HIP(hipMemcpy(host, t.ptr, nbytes, hipMemcpyDeviceToHost));
  CK_API_END
}

int ck_write_tensor(ck_engine* e, const char* name, const void* host, size_t nbytes) {
  CK_API_BEGIN
  CK_REQUIRE(e && name && host, "null argument");
  Tensor& t = e->tensor(name);
  CK_REQUIRE(nbytes <= t.nbytes, std::string("ck_write_tensor: size exceeds ") + name);
  if (t.param) {
    e->upload(name, host, nbytes);
  } else {
    CK_REQUIRE(t.ld == t.cols, std::string("ck_write_tensor: padded tensor ") + name);
    CK_HIP(hipStreamSynchronize(e->stream));
    CK_HIP(hipMemcpy(t.ptr, host, nbytes, hipMemcpyHostToDevice));
  }
  CK_API_END
}

int ck_gemv(const void* W, const float* x, const float* bias, float* y, int rows, int K, int ldw, int act,
            int rows_per_wg, void* stream) {
  CK_API_BEGIN
  launch_gemv(static_cast<const half_t*>(W), x, bias, y, rows, K, ldw, act, rows_per_wg, as_stream(stream));
  CK_API_END
}

int ck_gemm_workspace(int M, int N, int K, int b_kn, int* tile, int* split_k, size_t* ws_bytes) {
  CK_API_BEGIN
  GemmDesc d;
  d.M = M; d.N = N; d.K = K; d.b_kn = b_kn != 0;
  d.tile = tile ? *tile : 0;
  d.split = split_k ? *split_k : 0;
  const size_t f = gemm_plan(d);
  if (tile) *tile = d.tile;
  if (split_k) *split_k = d.split;
  if (ws_bytes) *ws_bytes = f * sizeof(float);
  CK_API_END
}

static void gemm_common(GemmDesc& d, const void* A, const void* B, void* C, const float* bias, int M, int N, int K,
                        long lda, long ldb, long ldc, int tile, int split_k, void* workspace, size_t ws_bytes) {
  d.A = static_cast<const half_t*>(A);
  d.B = static_cast<const half_t*>(B);
  d.C = C;
  d.bias = bias;
  d.M = M; d.N = N; d.K = K;
  d.lda = lda; d.ldb = ldb; d.ldc = ldc;
  d.tile = tile;
  d.split = split_k;
  d.ws = static_cast<float*>(workspace);
  d.ws_floats = ws_bytes / sizeof(float);
}

int ck_gemm(const void* A, const void* B, float* C, const float* bias, int M, int N, int K, long lda, long ldb,
            long ldc, int b_kn, int tile, int split_k, void* workspace, size_t ws_bytes, void* stream) {
  CK_API_BEGIN
  GemmDesc d;
  gemm_common(d, A, B, C, bias, M, N, K, lda, ldb, ldc, tile, split_k, workspace, ws_bytes);
  d.b_kn = b_kn != 0;
  d.epi = EPI_F32;
  launch_gemm(d, as_stream(stream));
  CK_API_END
}

int ck_gemm_epi(const void* A, const void* B, void* C, const float* bias, int M, int N, int K, long lda, long ldb,
                long ldc, int epi, int tile, int split_k, void* workspace, size_t ws_bytes, void* stream) {
  CK_API_BEGIN
  CK_REQUIRE(epi >= EPI_F16_BIAS && epi <= EPI_F32_RESID, "ck_gemm_epi: epi must be 1..4");
  GemmDesc d;
  gemm_common(d, A, B, C, bias, M, N, K, lda, ldb, ldc, tile, split_k, workspace, ws_bytes);
  d.epi = epi;
  launch_gemm(d, as_stream(stream));
  CK_API_END
}

int ck_wmma_rdna4(const uint16_t* fragA, const uint16_t* fragB, const float* fragC, float* fragD, int n_tiles,
                  void* stream) {
  CK_API_BEGIN
  launch_wmma_rdna4(fragA, fragB, fragC, fragD, n_tiles, as_stream(stream));
  CK_API_END
}

int ck_mfma_kat(int variant, const uint16_t* A, const uint16_t* B, float* D, void* stream) {
  CK_API_BEGIN
  launch_mfma_kat(variant, A, B, D, as_stream(stream));
  CK_API_END
}

int ck_pack_yuv(const uint8_t* Y, const uint8_t* U, const uint8_t* V, int H, int W, uint8_t* out, void* stream) {
  CK_API_BEGIN
  launch_yuv_to_channels(Y, U, V, H, W, out, as_stream(stream));
  CK_API_END
}

int ck_frames_to_tensor(const uint8_t* frame, int H, int W, uint8_t* out, void* stream) {
  CK_API_BEGIN
  launch_i420_to_channels(frame, H, W, out, as_stream(stream));
  CK_API_END
}

int ck_img_gather(const void* img, int A, int B, int lanes, int elem_bytes, const int32_t* yx, int n, void* out,
                  void* stream) {
  CK_API_BEGIN
  launch_img_gather(img, A, B, lanes, elem_bytes, yx, n, out, as_stream(stream));
  CK_API_END
}

int ck_warp_nv12(const uint8_t* frame, const uint8_t* big_frame, size_t frame_bytes, const float* tfm,
                 const float* big_tfm, int cam_w, int cam_h, int stride, int y_height, int model_w, int model_h,
                 int division, uint8_t* out, void* stream) {
  CK_API_BEGIN
  launch_warp_nv12(frame, big_frame, frame_bytes, tfm, big_tfm, cam_w, cam_h, stride, y_height, model_w, model_h,
                   division, out, as_stream(stream));
  CK_API_END
}

int ck_attention(const void* qk, const void* vt, void* out, int T, int n_heads, int head_dim, void* stream) {
  CK_API_BEGIN
  launch_attention(static_cast<const half_t*>(qk), static_cast<const half_t*>(vt), static_cast<half_t*>(out), T,
                   n_heads, head_dim, false, as_stream(stream));
  CK_API_END
}

int ck_layernorm(const float* x, const float* g, const float* b, void* out, int out_f16, int rows, int d, float eps,
                 void* stream) {
  CK_API_BEGIN
  launch_layernorm(x, g, b, out, out_f16 != 0, rows, d, eps, as_stream(stream));
  CK_API_END
}

}  // extern "C"
