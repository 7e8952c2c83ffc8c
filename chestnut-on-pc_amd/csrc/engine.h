// The per-frame engine: model spec, device tensors, the resolved frame plan
// and its hipGraph.  Replaces the reference's L4/L5 layers: pickle decode +
// queue allocation (run_pinned2.py:1346-1389) and the replay / CUDA-graph
// frame executor (run_pinned2.py:1391-1572).
#pragma once

#include <functional>
#include <map>
#include <string>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace ck {

struct Spec {
  std::string name;
  int img_h = 128, img_w = 256, n_frames = 2, fs = 4;
  int feat_len = 512, feat_hist = 24, desire_len = 8, desire_hist = 25;
  int hidden = 512, d = 0, n_heads = 0, head_dim = 0, n_layers = 0, d_ff = 0, temporal_dim = 0;
  float eps = 1e-5f;
  std::vector<int> stem;
  std::vector<std::pair<std::string, int>> outputs;
  // optional NV12 camera geometry (run_frame_nv12); width 0 = none
  int cam_w = 0, cam_h = 0, cam_stride = 0, cam_y_height = 0;
  // the warp's coordinate division: 0 "ieee" src_x / src_w, 1 "rcp" src_x * (1 / src_w)
  int cam_div = 0;
  // run the temporal and context GEMVs on a second stream beside the conv
  // stem (-1: the engine decides by model size, 0: off, 1: on)
  int overlap = -1;
  // run the policy inputs, the temporal GEMV and stem layer 1's im2col as one
  // launch (1, the default; 0: three launches; ignored when the context runs
  // on its own stream)
  int fuse_head = 1;
  // with the frame head: the context GEMV rides with the last stem layer's
  // split-K reduce launch (1, the default; 0: a launch of its own)
  int ride_context = 1;
  // attention and the output projection in one launch, the projection's
  // per-head f32 partials summed by the next LayerNorm (-1, the default: where
  // the heads fit the LayerNorm's 8 partials and the kernel takes the shape;
  // 0: off; 1: on, an error where it cannot be)
  int fuse_oproj = -1;
  // graph instantiation: 0 default; 1 upload the executable graph to the
  // engine stream (hipGraphUpload) before its first launch
  int graph_upload = 0;
  // optional per-plan-entry GEMM configuration {entry: [tile, split]} (A/B probes)
  std::vector<std::pair<std::string, std::pair<int, int>>> gemm_cfg;
};
Spec parse_spec(const std::string& json);

enum DType { DT_F32 = 0, DT_F16 = 1, DT_U8 = 2, DT_U32 = 3 };

struct Tensor {
  std::string name;
  void* ptr = nullptr;
  size_t nbytes = 0;     // logical bytes (what upload/read/write transfer)
  int dtype = DT_F32;
  long rows = 1, cols = 0, ld = 0;   // 2-D view for padded parameter layouts
  bool param = false;
};

struct Launch {
  std::string name;      // plan position, e.g. "blk3.qkv"
  std::string kernel;    // kernel family, e.g. "gemm_qkv"
  double flops = 0, bytes = 0;   // algorithmic work of one launch
  int branch = 0;        // 1: launched on the side stream (forked after the entries before it)
  bool join = false;     // the main stream waits for the side stream before this entry
  std::function<void(hipStream_t)> fn;
};

}  // namespace ck

struct ck_engine {
  ck::Spec sp;
  hipStream_t stream = nullptr;
  hipStream_t side = nullptr;                // second stream of a forked plan
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  std::vector<ck::Tensor> tensors;
  std::map<std::string, size_t> by_name;
  std::vector<ck::Launch> plan;
  bool use_graph = true;
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  size_t graph_nodes = 0;
  // run_frame's graph: the input copies from the pinned staging, the plan and
  // the output copy back, one launch per call (frame_launch replays `graph`)
  hipGraph_t graph_io = nullptr;
  hipGraphExec_t gexec_io = nullptr;
  float* ws = nullptr;
  size_t ws_floats = 0;
  // state hashing (ck_state_hashes): span table and per-span partials, built on first use
  std::vector<ck::HashSpan> hash_spans;
  ck::HashSpan* hash_spans_dev = nullptr;
  unsigned long long* hash_part_dev = nullptr;
  // output decode: per-head table (host + device copy), decoded-vector layout as JSON
  std::vector<ck::DecodeHead> dec_heads;
  ck::DecodeHead* dec_dev = nullptr;
  std::string dec_layout;
  int n_decoded = 0;
  uint8_t* h_warped = nullptr;   // pinned staging (outlives every async copy)
  float* h_packed = nullptr;
  float* h_out = nullptr;
  uint8_t* h_nv12 = nullptr;     // pinned staging of the two NV12 frames (camera specs only)
  float* h_tfm = nullptr;
  size_t nv12_bytes = 0;         // one NV12 frame
  // derived sizes
  int T = 0, n_spatial = 0, n_head_out = 0, n_out = 0, n_ctx = 0, ld_ctx = 0, packed_len = 0;
  size_t warped_bytes = 0;

  explicit ck_engine(const std::string& spec_json);
  ~ck_engine();

  ck::Tensor& tensor(const std::string& name);
  void* ptr(const std::string& name) { return tensor(name).ptr; }
  void upload(const std::string& name, const void* host, size_t nbytes);
  void run_frame(const uint8_t* warped, const float* packed, float* out);
  void run_frame_nv12(const uint8_t* frame, const uint8_t* big_frame, const float* tfm, const float* big_tfm,
                      const float* packed, float* out);
  void frame_launch();
  // timed: per plan entry, 1 = launch it with start/stop events appended to
  // events[i] (see LaunchTimer); null for plain launches and graph capture
  void launch_plan(const std::vector<char>* timed = nullptr,
                   std::vector<std::vector<std::pair<hipEvent_t, hipEvent_t>>>* events = nullptr);
  void capture();
  void capture_io();
  void drop_graph();
  void reset_state();
  void run_range(int first, int last);
  void kernel_times(float* ms, int n);
  float time_launches(const int* idx, int n, int reps);
  float time_in_frames(const int* idx, int n, int frames, float* per_entry_ms);
  // hash of every state tensor (non-parameter, allocation order), after the
  // work already queued on the engine stream
  void state_hashes(uint64_t* out, int n);

 private:
  void init();
  void release() noexcept;
  ck::Tensor& add_tensor(const std::string& name, size_t nbytes, int dtype, bool param, long rows = 1, long cols = 0,
                         long ld = 0);
  void build_params();
  void build_activations();
  void build_plan();
  void build_decode();
  void add(const std::string& name, const std::string& kernel, double flops, double bytes,
           std::function<void(hipStream_t)> fn);
  int add_gemm(const std::string& name, const std::string& kernel, ck::GemmDesc g);
};
