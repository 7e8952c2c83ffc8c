// Frame engine: spec -> parameter/activation tensors -> resolved launch plan
// -> hipGraph, one graph launch per frame.
//
// Reference structure being replaced (run_pinned2.py):
//   1346-1370  model load + graph flatten      -> build_params / build_plan
//   1372-1389  input queues and PACKED         -> ring buffers + staging tensors
//   1404-1420  first-frame plan recorder       -> the plan is resolved at create
//   1432-1502  capture on a stream, instantiate -> capture()
//   1503-1565  per-frame H2D, cuGraphLaunch, sync, D2H -> run_frame()
//   1513-1557  KSYNC per-launch event timing    -> kernel_times()
// Every launch of the plan has static device addresses, so the captured
// graph replays unchanged; the per-frame state that must move (queue
// positions, the recurrent hidden state) lives in device memory and is
// advanced by the plan's own kernels.
#include "engine.h"

#include <cmath>
#include <cstring>
#include <sstream>

#include "json.h"

namespace ck {

namespace {

long round_up(long v, long m) { return (v + m - 1) / m * m; }

// An integral JSON number within int range (what = the key, for the message).
int as_int(const JVal& v, const std::string& what) {
  CK_REQUIRE(v.kind == JVal::NUM, "spec: " + what + " must be a number");
  CK_REQUIRE(std::isfinite(v.num) && v.num == std::floor(v.num) && std::fabs(v.num) < 2147483648.0,
             "spec: " + what + " must be an integer");
  return (int)v.num;
}

int jint(const JVal& o, const char* k, int dflt, bool required = false) {
  const JVal* v = o.get(k);
  if (!v) {
    CK_REQUIRE(!required, std::string("spec: missing key ") + k);
    return dflt;
  }
  return as_int(*v, std::string("key ") + k);
}

}  // namespace

Spec parse_spec(const std::string& json) {
  JParser jp(json);
  JVal o = jp.parse();
  CK_REQUIRE(o.kind == JVal::OBJ, "spec: top level must be an object");
  Spec s;
  if (const JVal* v = o.get("name")) s.name = v->str;
  s.img_h = jint(o, "img_h", 128);
  s.img_w = jint(o, "img_w", 256);
  s.n_frames = jint(o, "n_frames", 2);
  s.fs = jint(o, "frame_skip", 4);
  s.feat_len = jint(o, "feat_len", 512);
  s.feat_hist = jint(o, "feat_hist", 24);
  s.desire_len = jint(o, "desire_len", 8);
  s.desire_hist = jint(o, "desire_hist", 25);
  s.hidden = jint(o, "hidden", 512);
  s.d = jint(o, "d_model", 0, true);
  s.n_heads = jint(o, "n_heads", 0, true);
  s.head_dim = jint(o, "head_dim", 0, true);
  s.n_layers = jint(o, "n_layers", 0, true);
  s.d_ff = jint(o, "d_ff", 0, true);
  s.temporal_dim = jint(o, "temporal_dim", 0, true);
  if (const JVal* v = o.get("ln_eps")) {
    CK_REQUIRE(v->kind == JVal::NUM && v->num > 0 && std::isfinite(v->num), "spec: ln_eps must be a positive number");
    s.eps = (float)v->num;
  }
  const JVal* st = o.get("stem");
  CK_REQUIRE(st && st->kind == JVal::ARR && !st->arr.empty(), "spec: stem must be a non-empty array");
  for (const auto& e : st->arr) s.stem.push_back(as_int(e, "stem width"));
  if (const JVal* ou = o.get("outputs")) {
    CK_REQUIRE(ou->kind == JVal::ARR, "spec: outputs must be an array of [name, size]");
    for (const auto& e : ou->arr) {
      CK_REQUIRE(e.kind == JVal::ARR && e.arr.size() == 2 && e.arr[0].kind == JVal::STR,
                 "spec: outputs entries are [name, size]");
      const int n = as_int(e.arr[1], "output size");
      CK_REQUIRE(n > 0, "spec: output sizes must be positive");
      s.outputs.emplace_back(e.arr[0].str, n);
    }
  }
  if (const JVal* cam = o.get("camera")) {
    CK_REQUIRE(cam->kind == JVal::OBJ, "spec: camera must be an object {width, height, stride, y_height}");
    s.cam_w = jint(*cam, "width", 0, true);
    s.cam_h = jint(*cam, "height", 0, true);
    s.cam_stride = jint(*cam, "stride", 0, true);
    s.cam_y_height = jint(*cam, "y_height", 0, true);
    if (const JVal* dv = cam->get("division")) {
      CK_REQUIRE(dv->kind == JVal::STR && (dv->str == "ieee" || dv->str == "rcp"),
                 "spec: camera.division must be \"ieee\" or \"rcp\"");
      s.cam_div = dv->str == "rcp";
    }
    CK_REQUIRE(s.cam_w > 0 && s.cam_h > 0 && s.cam_w % 2 == 0 && s.cam_h % 2 == 0 && s.cam_stride >= s.cam_w &&
                   s.cam_y_height >= s.cam_h,
               "spec: camera needs an even width and height, stride >= width, y_height >= height");
  }
  s.overlap = jint(o, "overlap_context", -1);
  s.fuse_head = jint(o, "fuse_head", 1);
  s.ride_context = jint(o, "ride_context", 1);
  s.fuse_oproj = jint(o, "fuse_oproj", -1);
  s.graph_upload = jint(o, "graph_upload", 0);
  if (const JVal* gc = o.get("gemm_config")) {
    CK_REQUIRE(gc->kind == JVal::OBJ, "spec: gemm_config must be an object {entry: [tile, split]}");
    for (const auto& kv : gc->obj) {
      CK_REQUIRE(kv.second.kind == JVal::ARR && kv.second.arr.size() == 2,
                 "spec: gemm_config entries are [tile, split]");
      s.gemm_cfg.push_back({kv.first, {as_int(kv.second.arr[0], "gemm_config tile"),
                                       as_int(kv.second.arr[1], "gemm_config split")}});
    }
  }
  // structural requirements of the kernels
  CK_REQUIRE(s.img_h > 0 && s.img_w > 0 && s.feat_len > 0 && s.feat_hist > 0 && s.desire_len > 0 &&
                 s.desire_hist > 0 && s.d > 0 && s.n_heads > 0 && s.n_layers > 0 && s.d_ff > 0 && s.temporal_dim > 0,
             "spec: sizes, counts and widths must be positive");
  for (int c : s.stem) CK_REQUIRE(c > 0, "spec: stem widths must be positive");
  CK_REQUIRE(s.head_dim == 64 || s.head_dim == 128, "spec: head_dim must be 64 or 128");
  CK_REQUIRE(s.feat_len % 8 == 0, "spec: feat_len must be a multiple of 8");
  CK_REQUIRE(s.n_frames == 2, "spec: n_frames must be 2 (two sampled frames per stream)");
  CK_REQUIRE(s.fs >= 1, "spec: frame_skip must be >= 1");
  CK_REQUIRE(s.d == s.n_heads * s.head_dim, "spec: d_model must equal n_heads * head_dim");
  CK_REQUIRE(s.hidden == s.feat_len, "spec: hidden must equal feat_len (prev_feat is the GRU state)");
  CK_REQUIRE(s.img_h % (1 << s.stem.size()) == 0 && s.img_w % (1 << s.stem.size()) == 0,
             "spec: image size must divide by 2^len(stem)");
  for (int c : s.stem) CK_REQUIRE(c % 8 == 0, "spec: stem channels must be multiples of 8");
  CK_REQUIRE(s.temporal_dim % 8 == 0 && s.d % 64 == 0 && s.d_ff % 64 == 0, "spec: widths must be multiples of 64");
  return s;
}

LaunchTimer& launch_timer() {
  static thread_local LaunchTimer t;
  return t;
}

}  // namespace ck

using namespace ck;

// A failure anywhere in set-up (a rejected gemm_config, an allocation)
// releases everything allocated so far before the exception leaves: a
// throwing constructor never runs the destructor.
ck_engine::ck_engine(const std::string& spec_json) : sp(parse_spec(spec_json)) {
  try {
    init();
  } catch (...) {
    release();
    throw;
  }
}

void ck_engine::init() {
  T = sp.stem.back();
  n_spatial = (sp.img_h >> sp.stem.size()) * (sp.img_w >> sp.stem.size());
  n_head_out = 0;
  for (auto& o : sp.outputs) n_head_out += o.second;
  n_out = n_head_out + sp.hidden;
  n_ctx = sp.temporal_dim + sp.desire_hist * sp.desire_len + 4;
  ld_ctx = (int)round_up(n_ctx, 8);
  packed_len = sp.desire_len + 4 + sp.feat_len;
  warped_bytes = 2ull * 6 * sp.img_h * sp.img_w;
  CK_REQUIRE(T % 64 == 0 && T <= 512, "spec: token count (last stem width) must be a multiple of 64, <= 512");
  CK_REQUIRE(2 * n_spatial % 64 == 0, "spec: token features must be a multiple of 64");
  CK_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  CK_HIP(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
  CK_HIP(hipEventCreateWithFlags(&ev_fork, hipEventDisableTiming));
  CK_HIP(hipEventCreateWithFlags(&ev_join, hipEventDisableTiming));
  build_params();
  build_activations();
  build_decode();
  build_plan();
  CK_HIP(hipHostMalloc((void**)&h_warped, warped_bytes, hipHostMallocDefault));
  CK_HIP(hipHostMalloc((void**)&h_packed, packed_len * sizeof(float), hipHostMallocDefault));
  CK_HIP(hipHostMalloc((void**)&h_out, n_out * sizeof(float), hipHostMallocDefault));
  if (sp.cam_w) {
    nv12_bytes = (size_t)sp.cam_stride * sp.cam_y_height + (size_t)(sp.cam_h / 2) * sp.cam_stride;
    add_tensor("nv12", 2 * nv12_bytes, DT_U8, false);
    add_tensor("tfm", 18 * sizeof(float), DT_F32, false);
    CK_HIP(hipHostMalloc((void**)&h_nv12, 2 * nv12_bytes, hipHostMallocDefault));
    CK_HIP(hipHostMalloc((void**)&h_tfm, 18 * sizeof(float), hipHostMallocDefault));
  }
  reset_state();
}

ck_engine::~ck_engine() { release(); }

void ck_engine::release() noexcept {
  if (stream) (void)hipStreamSynchronize(stream);
  if (side) (void)hipStreamSynchronize(side);
  drop_graph();
  for (auto& t : tensors)
    if (t.ptr) (void)hipFree(t.ptr);
  tensors.clear();
  by_name.clear();
  plan.clear();
  if (dec_dev) (void)hipFree(dec_dev);
  if (hash_spans_dev) (void)hipFree(hash_spans_dev);
  if (hash_part_dev) (void)hipFree(hash_part_dev);
  hash_spans_dev = nullptr;
  hash_part_dev = nullptr;
  hash_spans.clear();
  if (h_warped) (void)hipHostFree(h_warped);
  if (h_packed) (void)hipHostFree(h_packed);
  if (h_out) (void)hipHostFree(h_out);
  if (h_nv12) (void)hipHostFree(h_nv12);
  if (h_tfm) (void)hipHostFree(h_tfm);
  if (stream) (void)hipStreamDestroy(stream);
  if (side) (void)hipStreamDestroy(side);
  if (ev_fork) (void)hipEventDestroy(ev_fork);
  if (ev_join) (void)hipEventDestroy(ev_join);
  side = nullptr;
  ev_fork = ev_join = nullptr;
  dec_dev = nullptr;
  h_warped = nullptr; h_packed = nullptr; h_out = nullptr; h_nv12 = nullptr; h_tfm = nullptr;
  stream = nullptr;
  ws = nullptr;
}

Tensor& ck_engine::add_tensor(const std::string& name, size_t nbytes, int dtype, bool param, long rows, long cols,
                              long ld) {
  CK_REQUIRE(by_name.count(name) == 0, "duplicate tensor " + name);
  Tensor t;
  t.name = name;
  t.nbytes = nbytes;
  t.dtype = dtype;
  t.param = param;
  const size_t esz = dtype == DT_F16 ? 2 : dtype == DT_U8 ? 1 : 4;
  if (cols == 0) { rows = 1; cols = (long)(nbytes / esz); }
  if (ld == 0) ld = cols;
  t.rows = rows; t.cols = cols; t.ld = ld;
  const size_t alloc = std::max<size_t>(256, round_up((long)(rows * ld * esz), 256));
  CK_HIP(hipMalloc(&t.ptr, alloc));
  CK_HIP(hipMemset(t.ptr, 0, alloc));
  by_name[name] = tensors.size();
  tensors.push_back(t);
  return tensors.back();
}

Tensor& ck_engine::tensor(const std::string& name) {
  auto it = by_name.find(name);
  CK_REQUIRE(it != by_name.end(), "unknown tensor " + name);
  return tensors[it->second];
}

// Parameter table; must list the same names, shapes and dtypes as the
// Python side (chestnut/spec.py param_table).
void ck_engine::build_params() {
  const int d = sp.d, F = sp.d_ff, Hh = sp.hidden;
  auto f16 = [&](const std::string& n, long numel) { add_tensor(n, numel * 2, DT_F16, true); };
  auto f32 = [&](const std::string& n, long numel) { add_tensor(n, numel * 4, DT_F32, true); };
  int ci = 6 * sp.n_frames;
  for (size_t i = 0; i < sp.stem.size(); ++i) {
    const int co = sp.stem[i];
    const long K = 9L * ci;
    add_tensor("stem." + std::to_string(i) + ".w", 2L * co * K * 2, DT_F16, true, 2L * co, K, round_up(K, 64));
    f32("stem." + std::to_string(i) + ".b", 2L * co);
    ci = co;
  }
  f16("emb.w", (long)d * 2 * n_spatial);
  f32("emb.b", d);
  f16("pos", (long)T * d);
  f16("tmp.w", (long)sp.temporal_dim * sp.feat_hist * sp.feat_len);
  f32("tmp.b", sp.temporal_dim);
  add_tensor("ctx.w", (long)d * n_ctx * 2, DT_F16, true, d, n_ctx, ld_ctx);
  f32("ctx.b", d);
  for (int l = 0; l < sp.n_layers; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    f32(p + "ln1.g", d); f32(p + "ln1.b", d);
    f16(p + "qkv.w", 3L * d * d); f32(p + "qkv.b", 3L * d);
    f16(p + "o.w", (long)d * d); f32(p + "o.b", d);
    f32(p + "ln2.g", d); f32(p + "ln2.b", d);
    f16(p + "up.w", (long)F * d); f32(p + "up.b", F);
    f16(p + "down.w", (long)d * F); f32(p + "down.b", d);
  }
  f32("lnf.g", d); f32("lnf.b", d);
  f16("gru.wih", 3L * Hh * d); f32("gru.bih", 3L * Hh);
  f16("gru.whh", 3L * Hh * Hh); f32("gru.bhh", 3L * Hh);
  f16("head.w", (long)n_head_out * Hh); f32("head.b", n_head_out);
}

// Output decode table: each output head gets the Parser's treatment by name
// (parse_model_outputs.py:95-120); heads it does not parse (hidden_state,
// unknown names) pass through.  The decoded vector's layout is published as
// JSON (ck_decoded_layout).
void ck_engine::build_decode() {
  struct Rule {
    const char* name;
    int kind, width;
  };
  static const Rule rules[] = {
      {"pose", DEC_MDN, 0},           {"wide_from_device_euler", DEC_MDN, 0}, {"road_transform", DEC_MDN, 0},
      {"lane_lines", DEC_MDN, 0},     {"road_edges", DEC_MDN, 0},             {"plan", DEC_MDN, 0},
      {"lead", DEC_MDN, 0},           {"lane_lines_prob", DEC_SIGMOID, 0},    {"meta", DEC_SIGMOID, 0},
      {"lead_prob", DEC_SIGMOID, 0},  {"desire_pred", DEC_SOFTMAX, 8},        {"desire_state", DEC_SOFTMAX, 8}};
  // lead is multi-hypothesis (2 hypotheses, 3 selections) unless it holds
  // exactly 2 x 3 selections x 6 steps x 4 values (is_mhp, parse_model_outputs.py:88-93, 105-109)
  constexpr int LEAD_MDN_LEN = 2 * 3 * 6 * 4;
  std::vector<std::pair<std::string, int>> heads(sp.outputs);
  heads.push_back({"hidden_state", sp.hidden});
  std::ostringstream js;
  auto range = [&](const char* key, int a, int b) { js << "\"" << key << "\":[" << a << "," << b << "]"; };
  js << "{";
  int in_off = 0, out_off = 0;
  for (size_t k = 0; k < heads.size(); ++k) {
    const std::string& name = heads[k].first;
    DecodeHead h{};
    h.kind = DEC_RAW;
    h.in_off = in_off;
    h.len = heads[k].second;
    h.out_off = out_off;
    for (const Rule& r : rules)
      if (name == r.name) {
        h.kind = r.kind;
        h.width = r.width;
      }
    if (name == "lead" && h.len != LEAD_MDN_LEN) {
      h.kind = DEC_MHP;
      h.in_N = 2;
      h.out_N = 3;
    }
    int o = out_off;
    js << (k ? "," : "") << "\"" << name << "\":{";
    switch (h.kind) {
      case DEC_MDN:
        CK_REQUIRE(h.len >= 2, "decode: MDN head " + name + " needs at least 2 values");
        h.n = h.len / 2;
        js << "\"kind\":\"mdn\",\"n\":" << h.n << ",";
        range("mu", o, o + h.n);
        js << ",";
        range("std", o + h.n, o + 2 * h.n);
        o += 2 * h.n;
        break;
      case DEC_SIGMOID:
        js << "\"kind\":\"sigmoid\",";
        range("p", o, o + h.len);
        o += h.len;
        break;
      case DEC_SOFTMAX:
        CK_REQUIRE(h.len % h.width == 0, "decode: softmax head " + name + " is not a whole number of groups");
        js << "\"kind\":\"softmax\",\"width\":" << h.width << ",";
        range("p", o, o + h.len);
        o += h.len;
        break;
      case DEC_MHP: {
        const int L = h.len / h.in_N;
        CK_REQUIRE(h.len % h.in_N == 0 && L > h.out_N && (L - h.out_N) % 2 == 0,
                   "decode: multi-hypothesis head " + name + " does not split into [mu | std | weights]");
        h.n = (L - h.out_N) / 2;
        const int N = h.in_N, S = h.out_N, n = h.n;
        js << "\"kind\":\"mhp\",\"in_N\":" << N << ",\"out_N\":" << S << ",\"n\":" << n << ",";
        range("weights", o, o + N * S);
        o += N * S;
        js << ",";
        range("hyp_mu", o, o + N * n);
        o += N * n;
        js << ",";
        range("hyp_std", o, o + N * n);
        o += N * n;
        js << ",";
        range("mu", o, o + S * n);
        o += S * n;
        js << ",";
        range("std", o, o + S * n);
        o += S * n;
        break;
      }
      default:
        js << "\"kind\":\"raw\",";
        range("p", o, o + h.len);
        o += h.len;
        break;
    }
    js << "}";
    dec_heads.push_back(h);
    in_off += h.len;
    out_off = o;
  }
  js << "}";
  dec_layout = js.str();
  n_decoded = out_off;
  add_tensor("decoded", (size_t)n_decoded * 4, DT_F32, false);
  CK_HIP(hipMalloc((void**)&dec_dev, dec_heads.size() * sizeof(DecodeHead)));
  CK_HIP(hipMemcpy(dec_dev, dec_heads.data(), dec_heads.size() * sizeof(DecodeHead), hipMemcpyHostToDevice));
}

void ck_engine::build_activations() {
  const long HW = (long)sp.img_h * sp.img_w;
  const int d = sp.d;
  const int slots = sp.fs * (sp.n_frames - 1) + 1;
  add_tensor("warped", warped_bytes, DT_U8, false);
  add_tensor("packed", packed_len * 4, DT_F32, false);
  add_tensor("out", n_out * 4, DT_F32, false);
  add_tensor("counter", 4, DT_U32, false);
  add_tensor("img_ring", 2L * slots * 6 * HW, DT_U8, false);
  add_tensor("feat_ring", (long)sp.fs * sp.feat_hist * sp.feat_len * 4, DT_F32, false);
  add_tensor("desire_ring", (long)sp.fs * sp.desire_hist * sp.desire_len * 4, DT_F32, false);
  add_tensor("img", 2L * 6 * sp.n_frames * HW, DT_U8, false);
  add_tensor("feat_buf", (long)sp.feat_hist * sp.feat_len * 4, DT_F32, false);
  add_tensor("ctx_in", (long)ld_ctx * 4, DT_F32, false);
  long patches = 0;
  int H = sp.img_h, W = sp.img_w, C = 6 * sp.n_frames;
  for (size_t i = 0; i < sp.stem.size(); ++i) {
    const int Ho = (H - 1) / 2 + 1, Wo = (W - 1) / 2 + 1;
    patches = std::max(patches, 2L * Ho * Wo * round_up(9L * C, 64));
    add_tensor("stem." + std::to_string(i) + ".out", 2L * Ho * Wo * sp.stem[i] * 2, DT_F16, false);
    H = Ho; W = Wo; C = sp.stem[i];
  }
  add_tensor("patches", patches * 2, DT_F16, false);
  add_tensor("zero16", 256, DT_F16, false);   // never written: the implicit conv's border and K-padding source
  add_tensor("tokens", (long)T * 2 * n_spatial * 2, DT_F16, false);
  add_tensor("ctx", (long)d * 4, DT_F32, false);
  add_tensor("x", (long)T * d * 4, DT_F32, false);
  add_tensor("h16", (long)T * d * 2, DT_F16, false);
  add_tensor("qk", (long)T * 2 * d * 2, DT_F16, false);
  add_tensor("vt", (long)d * T * 2, DT_F16, false);
  add_tensor("att", (long)T * d * 2, DT_F16, false);
  add_tensor("u", (long)T * sp.d_ff * 2, DT_F16, false);
  add_tensor("xf", (long)T * d * 4, DT_F32, false);
  add_tensor("pooled", (long)d * 4, DT_F32, false);
  add_tensor("gi", 3L * sp.hidden * 4, DT_F32, false);
  add_tensor("gh", 3L * sp.hidden * 4, DT_F32, false);
  add_tensor("h_new", (long)sp.hidden * 4, DT_F32, false);
}

void ck_engine::add(const std::string& name, const std::string& kernel, double flops, double bytes,
                    std::function<void(hipStream_t)> fn) {
  Launch l;
  l.name = name;
  l.kernel = kernel;
  l.flops = flops;
  l.bytes = bytes;
  l.fn = std::move(fn);
  plan.push_back(std::move(l));
}

int ck_engine::add_gemm(const std::string& name, const std::string& kernel, GemmDesc g) {
  for (const auto& c : sp.gemm_cfg)
    if (c.first == name) {
      g.tile = c.second.first;
      g.split = c.second.second;
    }
  const size_t need = gemm_plan(g);
  ws_floats = std::max(ws_floats, need);
  const double M = g.M, N = g.N, K = g.K, B = g.batch;
  const bool out32 = g.epi == EPI_F32 || g.epi == EPI_F32_RESID;
  // A of an implicit conv: the input activation, each element read once
  const double a_elems = g.conv_c > 0 ? (double)g.conv_h * g.conv_w * g.conv_c : M * K;
  double bytes = B * (a_elems + N * K) * 2 + B * M * N * (out32 ? 4 : 2) + (g.bias ? B * N * 4 : 0);
  if (g.epi == EPI_F32_RESID) bytes += B * M * N * 4;
  std::string kern = kernel + (g.split > 1 ? "+splitk" + std::to_string(g.split) : "");
  double flops = 2.0 * M * N * K * B;
  if (g.rider.rows > 0) {   // the GEMV riding with the split-K reduce
    kern += "+gemv";
    flops += 2.0 * g.rider.rows * g.rider.K;
    bytes += 2.0 * g.rider.rows * g.rider.K + 4.0 * g.rider.K + 8.0 * g.rider.rows;
  }
  ck_engine* self = this;
  add(name, kern, flops, bytes, [self, g](hipStream_t s) {
    GemmDesc d = g;
    d.ws = self->ws;
    d.ws_floats = self->ws_floats;
    launch_gemm(d, s);
  });
  return g.split;
}

void ck_engine::build_plan() {
  plan.clear();
  const int d = sp.d, F = sp.d_ff, Hh = sp.hidden, dl = sp.desire_len;
  const long HW = (long)sp.img_h * sp.img_w;
  // The GEMVs load their weights non-temporally unless the whole model's
  // parameters fit comfortably in the 256 MB Infinity Cache, where the
  // default policy keeps them from one frame to the next (39M model: -1.1%
  // per frame; the 1B model's 2 GB stream either way and gain from it).
  size_t param_bytes = 0;
  for (const auto& t : tensors)
    if (t.param) param_bytes += t.nbytes;
  const bool stream_w = param_bytes > (size_t(128) << 20);
  auto h16 = [&](const std::string& n) { return static_cast<half_t*>(ptr(n)); };
  auto f32 = [&](const std::string& n) { return static_cast<float*>(ptr(n)); };

  const bool overlap = sp.overlap >= 0 ? sp.overlap != 0 : false;
  const int Kt = sp.feat_hist * sp.feat_len, Td = sp.temporal_dim;
  const double tmp_flops = 2.0 * Td * Kt, tmp_bytes = (double)Td * Kt * 2 + Kt * 4 + Td * 8;
  // The frame head: the policy inputs, the temporal GEMV and stem layer 1's
  // im2col in one launch (launch_frame_head), none of them waiting on
  // another: two dependent dispatches fewer (whole frames in alternating
  // processes: 39M -1.2 to -2.2%, 1B -0.4%; bit-identical).
  const bool head = !overlap && sp.fuse_head != 0;
  // 1. policy inputs: queue push + sample (compile_modeld.py:198-212)
  {
    QueueDims q{sp.img_h, sp.img_w, sp.fs, sp.fs * (sp.n_frames - 1) + 1, sp.feat_len, sp.feat_hist, sp.desire_len,
                sp.desire_hist};
    const uint8_t* warped = static_cast<uint8_t*>(ptr("warped"));
    const float* packed = f32("packed");
    const unsigned* counter = static_cast<unsigned*>(ptr("counter"));
    uint8_t* ring = static_cast<uint8_t*>(ptr("img_ring"));
    float* fr = f32("feat_ring");
    float* dr = f32("desire_ring");
    uint8_t* img = static_cast<uint8_t*>(ptr("img"));
    float* fb = f32("feat_buf");
    float* tail = f32("ctx_in") + sp.temporal_dim;
    const double bytes = 10.0 * 6 * HW + 2.0 * sp.feat_hist * sp.feat_len * 4 + 2.0 * sp.feat_len * 4;
    if (head) {
      const half_t* tw = h16("tmp.w");
      const float* tb = f32("tmp.b");
      float* cin = f32("ctx_in");
      half_t* patches = h16("patches");
      const int C0 = 6 * sp.n_frames, Kp0 = (int)round_up(9L * C0, 64);
      const int Ho0 = (sp.img_h - 1) / 2 + 1, Wo0 = (sp.img_w - 1) / 2 + 1;
      const double im2col_bytes = 2.0 * Ho0 * Wo0 * Kp0 * 2 + 2.0 * C0 * HW;
      const int slots = frame_head_slots(Kt, stream_w);   // a device query: here, never under graph capture
      add("inputs", "frame_head", tmp_flops, bytes + tmp_bytes + im2col_bytes, [=](hipStream_t s) {
        launch_frame_head(q, warped, packed, counter, ring, fr, dr, img, fb, tail, tw, tb, cin, Td, GEMV_GELU, stream_w,
                          patches, Kp0, slots, s);
      });
    } else {
      add("inputs", "policy_inputs", 0, bytes, [=](hipStream_t s) {
        launch_policy_inputs(q, warped, packed, counter, ring, fr, dr, img, fb, tail, s);
      });
    }
  }
  // The temporal and context GEMVs depend only on the feature queue: with
  // `overlap` they run on a second stream forked after the inputs, beside
  // the conv stem, and the embedding waits for them.
  // With the frame head the context GEMV rides with the split-K reduce of the
  // last stem layer (its inputs are ready after the head, the embedding needs
  // its output): set in the stem loop below.  One launch fewer: 39M frame
  // -1.0%, 1B unchanged within noise (bit-identical).
  bool ctx_rides = false;
  auto add_context = [&](int branch) {
    if (ctx_rides) return;
    if (!head) {
      const half_t* tw = h16("tmp.w");
      const float* tb = f32("tmp.b");
      const float* fbuf = f32("feat_buf");
      float* cin = f32("ctx_in");
      add("temporal", "gemv", tmp_flops, tmp_bytes, [=](hipStream_t s) {
        launch_gemv(tw, fbuf, tb, cin, Td, Kt, Kt, GEMV_GELU, 0, s, stream_w);
      });
      plan.back().branch = branch;
    }
    float* cin = f32("ctx_in");
    const half_t* cw = h16("ctx.w");
    const float* cb = f32("ctx.b");
    float* ctx = f32("ctx");
    const int ldc = ld_ctx;
    add("context", "gemv", 2.0 * d * ldc, (double)d * ldc * 2 + ldc * 4 + d * 8, [=](hipStream_t s) {
      launch_gemv(cw, cin, cb, ctx, d, ldc, ldc, GEMV_NONE, 0, s, stream_w);
    });
    plan.back().branch = branch;
  };
  if (overlap) add_context(1);
  bool tokens_fused = false;
  // 2. conv stem, both streams batched.  Layer 0 (u8 image, 12 channels):
  // im2col with zero-border image reads + MFMA GEMM.  Later layers (f16,
  // power-of-two channels): implicit GEMM, the conv GEMM gathers its A chunks
  // from the previous layer's output (no patch matrix, no im2col launch),
  // unless the spec pins the layer to a tile without that A path.
  {
    int H = sp.img_h, W = sp.img_w, C = 6 * sp.n_frames;
    for (size_t i = 0; i < sp.stem.size(); ++i) {
      const std::string si = std::to_string(i);
      const int Co = sp.stem[i];
      const int Ho = (H - 1) / 2 + 1, Wo = (W - 1) / 2 + 1;
      const int Kp = (int)round_up(9L * C, 64);
      half_t* patches = h16("patches");
      const double pbytes = 2.0 * Ho * Wo * Kp * 2;
      int tile = 0, cfg_split = -1;
      for (const auto& c : sp.gemm_cfg)
        if (c.first == "stem" + si + ".conv") { tile = c.second.first; cfg_split = c.second.second; }
      const bool implicit = i > 0 && C >= 8 && (C & (C - 1)) == 0 && (tile <= 8 || tile == 15);
      // default 64x64 tiles (one K-group for the implicit layers), and for
      // 18 or more K-steps a split that leaves 3 steps per workgroup: chosen
      // on whole 1B frames over every candidate (python -m chestnut.tune),
      // where the stem's weights arrive cold and a few long K chains are
      // latency-bound (K = 1152: split 6, K = 2304: split 12, -0.45% per
      // frame over unsplit two-K-group tiles)
      const int ksteps = Kp / 64;
      const int stem_split = (ksteps >= 18 && ksteps % 3 == 0) ? std::min(16, ksteps / 3) : 1;
      const int stem_tile = i == 0 ? 4 : 8;
      if (implicit) {
        GemmDesc g;
        g.A = h16("stem." + std::to_string(i - 1) + ".out"); g.sA = (long)H * W * C;
        g.conv_c = C; g.conv_h = H; g.conv_w = W; g.zero16 = h16("zero16");
        g.B = h16("stem." + si + ".w"); g.ldb = Kp; g.sB = (long)Co * Kp;
        g.C = ptr("stem." + si + ".out"); g.ldc = Co; g.sC = (long)Ho * Wo * Co;
        g.bias = f32("stem." + si + ".b"); g.sBias = Co;
        g.M = Ho * Wo; g.N = Co; g.K = Kp; g.batch = 2; g.epi = EPI_F16_BIAS_RELU;
        g.tile = stem_tile; g.split = stem_split;
        // last layer with split-K: its reduce stores the channels-as-tokens
        // transpose F[c][s*NS + p] directly (no separate tokens launch)
        const int eff_split = cfg_split >= 0 ? cfg_split : stem_split;
        if (i + 1 == sp.stem.size() && eff_split > 1 && Co == T && Ho * Wo == n_spatial) {
          g.c_nm = 1; g.C = ptr("tokens"); g.ldc = 2L * n_spatial; g.sC = n_spatial;
          tokens_fused = true;
        }
        if (i + 1 == sp.stem.size() && eff_split > 1 && head && sp.ride_context != 0) {
          g.rider.W = h16("ctx.w"); g.rider.x = f32("ctx_in"); g.rider.bias = f32("ctx.b"); g.rider.y = f32("ctx");
          g.rider.rows = d; g.rider.K = ld_ctx; g.rider.stream = stream_w;
          ctx_rides = true;
        }
        add_gemm("stem" + si + ".conv", "gemm_conv_relu_implicit", g);
        H = Ho; W = Wo; C = Co;
        continue;
      }
      if (i == 0 && head) {
        // the patches come from the frame head
      } else if (i == 0) {
        const uint8_t* img = static_cast<uint8_t*>(ptr("img"));
        add("stem0.im2col", "im2col_u8", 0, pbytes + 2.0 * C * HW, [=](hipStream_t s) {
          launch_im2col_u8(img, 2, C, H, W, patches, Kp, s);
        });
      } else {
        const half_t* prev = h16("stem." + std::to_string(i - 1) + ".out");
        add("stem" + si + ".im2col", "im2col_f16", 0, pbytes + 2.0 * H * W * C * 2, [=](hipStream_t s) {
          launch_im2col_f16(prev, 2, C, H, W, patches, Kp, s);
        });
      }
      GemmDesc g;
      g.A = patches; g.lda = Kp; g.sA = (long)Ho * Wo * Kp;
      g.B = h16("stem." + si + ".w"); g.ldb = Kp; g.sB = (long)Co * Kp;
      g.C = ptr("stem." + si + ".out"); g.ldc = Co; g.sC = (long)Ho * Wo * Co;
      g.bias = f32("stem." + si + ".b"); g.sBias = Co;
      g.M = Ho * Wo; g.N = Co; g.K = Kp; g.batch = 2; g.epi = EPI_F16_BIAS_RELU;
      g.tile = stem_tile; g.split = stem_split;
      add_gemm("stem" + si + ".conv", "gemm_conv_relu", g);
      H = Ho; W = Wo; C = Co;
    }
  }
  // 3. tokens, temporal context, embedding
  {
    const half_t* so = h16("stem." + std::to_string(sp.stem.size() - 1) + ".out");
    half_t* tok = h16("tokens");
    const int ns = n_spatial, C5 = T;
    if (!tokens_fused)
      add("tokens", "tokens", 0, 2.0 * 2 * ns * C5 * 2, [=](hipStream_t s) { launch_tokens(so, ns, C5, tok, s); });
    if (!overlap) add_context(0);
    float* ctx = f32("ctx");
    const half_t* pos = h16("pos");
    const float* eb = f32("emb.b");
    float* x = f32("x");
    // X0 = F W_emb^T + b + pos + ctx, all in the GEMM's epilogue
    GemmDesc g;
    g.A = tok; g.lda = 2 * ns;
    g.B = h16("emb.w"); g.ldb = 2 * ns;
    g.C = x; g.ldc = d; g.bias = eb; g.pos = pos; g.ctx = ctx;
    g.M = T; g.N = d; g.K = 2 * ns; g.epi = EPI_EMBED;
    g.tile = 4;   // 64x64: a one- or two-step GEMM whose time is its epilogue, spread over 4x the workgroups
    add_gemm("embed", "gemm_embed", g);
    plan.back().join = overlap;
  }
  // 4. transformer blocks.  The two residual GEMMs (attention output, MLP
  // down) split K and leave f32 partials in the workspace; the LayerNorm that
  // follows each of them adds partials + bias into x before normalising.
  // Tiles and splits were chosen on whole frames of the 1B model (a GEMM's
  // time inside the frame differs from its time in a loop of its own):
  //   QKV: 128x96 (below), MLP up: 128x128, one K-group;  O-proj: 64x128,
  //   two K-groups, split to fill 256 workgroups (128x64 until the
  //   cache-policy changes of the stores and weight loads; retuned: -1.5% of
  //   the 1B frame);  MLP down: 128x128, one K-group, split to fill 256.
  //   GEMMs whose 128x128 tiles would leave most CUs idle (fewer than 64
  //   tiles: the 39M model's 256 tokens x d = 512) run on smaller tiles
  //   (below; whole 39M frames on 64x64 tiles: 0.264 -> 0.209 ms).
  auto small = [&](int N) { return (long)ceil_div(T, 128) * ceil_div(N, 128) < 64; };
  auto resid_split = [&](int M, int N, int K, int bm, int bn, int kmult, int kmin) {
    const long tiles = (long)ceil_div(M, bm) * ceil_div(N, bn);
    int s = 1;
    while (tiles * s * 2 <= 256 && K % (kmult * s * 2) == 0 && K / (s * 2) >= kmin) s *= 2;
    return s;
  };
  // QKV on the 128x96 tile (gemm tile 10) where 128x128 tiles leave CUs idle
  // and 128x96 ones still fit one wave of 256 CUs: every CU streams 7/8 of
  // the bytes (1B: 192 -> 256 workgroups, QKV 22.96 -> 21.44 us, frame -1.9%)
  const long qt128 = (long)(T / 128) * (3 * d / 128), qt96 = (long)(T / 128) * (3 * d / 96);
  const bool qkv96 = T % 128 == 0 && (3 * d) % 96 == 0 && qt128 < 256 && qt96 <= 256 && sp.head_dim >= 32;
  // Small models: QKV and MLP-up on 32x64 tiles (gemm tile 15, two waves)
  // where that grid still fits one wave of 256 workgroups, MLP-down on 64x64
  // tiles with two K-groups, split to 512-wide K slices (39M frames, one
  // process, alternating engines: 0.1866 -> 0.1816 ms; each alone less).
  auto fits32 = [&](int N) { return (long)ceil_div(T, 32) * ceil_div(N, 64) <= 256; };
  const int tile_o = small(d) ? 8 : 3, tile_dn = small(d) ? 4 : 5;
  const int tile_qkv = small(3 * d) ? (fits32(3 * d) && sp.head_dim >= 32 ? 15 : 8) : qkv96 ? 10 : 5;
  const int tile_up = small(F) ? (fits32(F) ? 15 : 8) : 5;
  const int s_o = small(d) ? resid_split(T, d, d, 64, 64, 64, 256) : resid_split(T, d, d, 64, 128, 128, 512);
  const int s_dn = small(d) ? resid_split(T, d, F, 64, 64, 128, 512) : resid_split(T, d, F, 128, 128, 128, 512);
  ck_engine* self = this;
  const long part_stride = (long)T * d;
  // attention + O-projection in one launch: one partial plane per head
  const bool oproj_ok = attention_oproj_tiles(T, sp.n_heads, sp.head_dim) > 0 && sp.n_heads <= 8;
  CK_REQUIRE(sp.fuse_oproj != 1 || oproj_ok,
             "spec: fuse_oproj needs at most 8 heads and a shape the fused attention takes");
  const bool fuse_o = sp.fuse_oproj == 1 || (sp.fuse_oproj < 0 && oproj_ok);
  if (fuse_o) ws_floats = std::max(ws_floats, (size_t)sp.n_heads * T * d);
  const float* pend_bias = nullptr;   // bias of the GEMM whose partials the next LN must add
  int pend_split = 0;
  auto add_ln = [&](const std::string& name, const float* g, const float* bb, void* out, bool f16) {
    float* x = f32("x");
    const float* rb = pend_bias;
    const int ns = pend_split;
    const int Tt = T;
    const float eps = sp.eps;
    const double bytes = (double)Tt * d * (4 + 4 + (f16 ? 2 : 4)) + (ns ? (double)Tt * d * 4 * ns : 0);
    add(name, ns ? (f16 ? "add_layernorm_f16" : "add_layernorm_f32") : (f16 ? "layernorm_f16" : "layernorm_f32"), 0,
        bytes, [=](hipStream_t s) {
          launch_add_layernorm(x, ns ? self->ws : nullptr, ns, part_stride, rb, g, bb, out, f16, Tt, d, eps, s);
        });
    pend_bias = nullptr;
    pend_split = 0;
  };
  for (int l = 0; l < sp.n_layers; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    const std::string b = "blk" + std::to_string(l) + ".";
    half_t* hb = h16("h16");
    add_ln(b + "ln1", f32(p + "ln1.g"), f32(p + "ln1.b"), hb, true);
    GemmDesc q;
    q.A = hb; q.lda = d; q.B = h16(p + "qkv.w"); q.ldb = d; q.C = ptr("qk"); q.ldc = 2 * d;
    q.bias = f32(p + "qkv.b"); q.M = T; q.N = 3 * d; q.K = d; q.epi = EPI_QKV_FRAG;
    q.vt = h16("vt"); q.qk_cols = 2 * d; q.vt_ld = T; q.head_dim = sp.head_dim;
    q.tile = tile_qkv; q.split = 1;   // 128x96 or 128x128 tiles (32x64 or 64x64 when small), one K-group
    add_gemm(b + "qkv", "gemm_qkv", q);
    const half_t* qk = h16("qk");
    const half_t* vt = h16("vt");
    half_t* att = h16("att");
    const int nh = sp.n_heads, hd = sp.head_dim, Tt = T;
    if (fuse_o) {
      // the head-h plane of the O-projection comes out of head h's attention
      // workgroups; the LayerNorm adds the n_heads planes in head order
      const half_t* wo = h16(p + "o.w");
      add(b + "attn", "attention_oproj", 4.0 * Tt * Tt * d + 2.0 * Tt * d * d,
          (double)Tt * d * 2 * 3 + (double)d * d * 2 + (double)nh * Tt * d * 4,
          [=](hipStream_t s) { launch_attention_oproj(qk, vt, wo, self->ws, Tt, nh, hd, s); });
      pend_split = nh;
    } else {
      add(b + "attn", "attention", 4.0 * Tt * Tt * d, (double)Tt * d * 2 * 4, [=](hipStream_t s) {
        launch_attention(qk, vt, att, Tt, nh, hd, true, s);
      });
      GemmDesc o;
      o.A = att; o.lda = d; o.B = h16(p + "o.w"); o.ldb = d;
      o.M = T; o.N = d; o.K = d; o.epi = EPI_PARTIALS; o.tile = tile_o; o.split = s_o;   // 64x128 (64x64 when small)
      pend_split = add_gemm(b + "o", "gemm_partials", o);   // the split actually used (gemm_config may set it)
    }
    pend_bias = f32(p + "o.b");
    add_ln(b + "ln2", f32(p + "ln2.g"), f32(p + "ln2.b"), hb, true);
    GemmDesc up;
    up.A = hb; up.lda = d; up.B = h16(p + "up.w"); up.ldb = d; up.C = ptr("u"); up.ldc = F;
    up.bias = f32(p + "up.b"); up.M = T; up.N = F; up.K = d; up.epi = EPI_F16_BIAS_GELU;
    up.tile = tile_up; up.split = 1;  // 128x128 tiles (32x64 or 64x64 when small), one K-group
    add_gemm(b + "up", "gemm_gelu", up);
    GemmDesc dn;
    dn.A = h16("u"); dn.lda = F; dn.B = h16(p + "down.w"); dn.ldb = F;
    dn.M = T; dn.N = d; dn.K = F; dn.epi = EPI_PARTIALS; dn.tile = tile_dn; dn.split = s_dn;
    pend_split = add_gemm(b + "down", "gemm_partials", dn);
    pend_bias = f32(p + "down.b");
  }
  // 5. final LN (adds the last block's MLP partials) + pool, GRU, heads, tick
  {
    float* xf = f32("xf");
    float* pooled = f32("pooled");
    const int Tt = T;
    add_ln("final.ln", f32("lnf.g"), f32("lnf.b"), xf, false);
    add("final.pool", "colmean", 0, (double)Tt * d * 4, [=](hipStream_t s) { launch_colmean(xf, pooled, Tt, d, s); });
    const float* hprev = f32("packed") + dl + 4;
    float* gi = f32("gi");
    float* gh = f32("gh");
    const half_t* wih = h16("gru.wih");
    const half_t* whh = h16("gru.whh");
    const float* bih = f32("gru.bih");
    const float* bhh = f32("gru.bhh");
    // gi = W_ih pooled + b_ih and gh = W_hh h_prev + b_hh: one launch
    add("gru", "gemv2", 2.0 * 3 * Hh * (d + Hh), 3.0 * Hh * (d + Hh) * 2, [=](hipStream_t s) {
      launch_gemv2(wih, pooled, bih, gi, 3 * Hh, d, whh, hprev, bhh, gh, 3 * Hh, Hh, s, stream_w);
    });
    // heads on the new hidden state; the GRU update is computed inside the
    // GEMV, which also stores h to h_new and to the output's hidden_state slice
    float* out = f32("out");
    float* hn = f32("h_new");
    const int nho = n_head_out;
    const half_t* hw = h16("head.w");
    const float* hbias = f32("head.b");
    add("heads", "gemv_gru", 2.0 * nho * Hh, (double)nho * Hh * 2 + 7.0 * Hh * 4, [=](hipStream_t s) {
      launch_gemv_gru(hw, hbias, out, nho, gi, gh, hprev, hn, out + nho, Hh, s, stream_w);
    });
    // the Parser's decode, and in the same launch the end-of-frame tick:
    // queue counter + 1, h_new -> packed prev_feat (read by the next frame)
    float* dec = f32("decoded");
    const DecodeHead* dd = dec_dev;
    const int ndh = (int)dec_heads.size();
    unsigned* counter = static_cast<unsigned*>(ptr("counter"));
    float* feat = f32("packed") + dl + 4;
    add("decode", "decode", 0, (double)(n_out + n_decoded) * 4 + 8.0 * Hh, [=](hipStream_t s) {
      launch_decode(out, dec, dd, ndh, s, counter, hn, feat, Hh);
    });
  }
  // the split-K workspace is an ordinary activation tensor ("ws"), so state
  // snapshots (probes) see the partials a residual LayerNorm consumes
  if (ws_floats) ws = static_cast<float*>(add_tensor("ws", ws_floats * sizeof(float), DT_F32, false).ptr);
}

void ck_engine::upload(const std::string& name, const void* host, size_t nbytes) {
  Tensor& t = tensor(name);
  CK_REQUIRE(nbytes == t.nbytes, "upload " + name + ": expected " + std::to_string(t.nbytes) + " bytes, got " +
                                     std::to_string(nbytes));
  if (t.ld == t.cols) {
    CK_HIP(hipMemcpy(t.ptr, host, nbytes, hipMemcpyHostToDevice));
  } else {
    const size_t esz = t.dtype == DT_F16 ? 2 : t.dtype == DT_U8 ? 1 : 4;
    CK_HIP(hipMemcpy2D(t.ptr, t.ld * esz, host, t.cols * esz, t.cols * esz, t.rows, hipMemcpyHostToDevice));
  }
}

void ck_engine::drop_graph() {
  if (gexec) (void)hipGraphExecDestroy(gexec);
  if (graph) (void)hipGraphDestroy(graph);
  if (gexec_io) (void)hipGraphExecDestroy(gexec_io);
  if (graph_io) (void)hipGraphDestroy(graph_io);
  gexec = nullptr;
  graph = nullptr;
  gexec_io = nullptr;
  graph_io = nullptr;
  graph_nodes = 0;
}

// The plan in order on the engine stream; entries marked `branch` go to the
// side stream, forked from the engine stream at the first of them, and the
// engine stream waits for the side stream at the next entry marked `join`
// (or at the end).  The same calls serve eager frames and graph capture,
// where the fork and join become graph edges.
void ck_engine::launch_plan(const std::vector<char>* timed,
                            std::vector<std::vector<std::pair<hipEvent_t, hipEvent_t>>>* events) {
  bool forked = false, pending = false;
  LaunchTimer& lt = launch_timer();
  auto run = [&](size_t i, hipStream_t s) {
    if (!timed || !(*timed)[i]) {
      plan[i].fn(s);
      return;
    }
    lt.events.clear();
    lt.on = true;
    try {
      plan[i].fn(s);
    } catch (...) {
      lt.on = false;
      for (auto& e : lt.events) (*events)[i].push_back(e);
      lt.events.clear();
      throw;
    }
    lt.on = false;
    for (auto& e : lt.events) (*events)[i].push_back(e);
    lt.events.clear();
  };
  for (size_t i = 0; i < plan.size(); ++i) {
    const Launch& l = plan[i];
    if (l.branch) {
      if (!forked) {
        CK_HIP(hipEventRecord(ev_fork, stream));
        CK_HIP(hipStreamWaitEvent(side, ev_fork, 0));
        forked = true;
      }
      run(i, side);
      pending = true;
      continue;
    }
    if (pending && l.join) {
      CK_HIP(hipEventRecord(ev_join, side));
      CK_HIP(hipStreamWaitEvent(stream, ev_join, 0));
      pending = false;
    }
    run(i, stream);
  }
  if (pending) {
    CK_HIP(hipEventRecord(ev_join, side));
    CK_HIP(hipStreamWaitEvent(stream, ev_join, 0));
  }
}

void ck_engine::capture() {
  drop_graph();
  CK_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
  try {
    launch_plan();
  } catch (...) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(stream, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  CK_HIP(hipStreamEndCapture(stream, &graph));
  CK_HIP(hipGraphGetNodes(graph, nullptr, &graph_nodes));
  CK_HIP(hipGraphInstantiate(&gexec, graph, nullptr, nullptr, 0));
  if (sp.graph_upload) {
    CK_HIP(hipGraphUpload(gexec, stream));
    CK_HIP(hipStreamSynchronize(stream));
  }
}

// The same plan between the copies of run_frame: pinned staging -> warped and
// packed, the plan, out -> pinned staging.  The staging addresses are fixed
// for the engine's life, so the copy nodes are recorded once; each call
// fills the staging before the launch and reads it after the sync.
void ck_engine::capture_io() {
  if (!gexec) capture();
  CK_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
  try {
    CK_HIP(hipMemcpyAsync(ptr("warped"), h_warped, warped_bytes, hipMemcpyHostToDevice, stream));
    CK_HIP(hipMemcpyAsync(ptr("packed"), h_packed, packed_len * sizeof(float), hipMemcpyHostToDevice, stream));
    launch_plan();
    CK_HIP(hipMemcpyAsync(h_out, ptr("out"), n_out * sizeof(float), hipMemcpyDeviceToHost, stream));
  } catch (...) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(stream, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  CK_HIP(hipStreamEndCapture(stream, &graph_io));
  CK_HIP(hipGraphInstantiate(&gexec_io, graph_io, nullptr, nullptr, 0));
  if (sp.graph_upload) {
    CK_HIP(hipGraphUpload(gexec_io, stream));
    CK_HIP(hipStreamSynchronize(stream));
  }
}

void ck_engine::frame_launch() {
  if (use_graph) {
    if (!gexec) capture();
    CK_HIP(hipGraphLaunch(gexec, stream));
  } else {
    launch_plan();
  }
}

void ck_engine::run_frame(const uint8_t* warped, const float* packed, float* out) {
  std::memcpy(h_warped, warped, warped_bytes);
  std::memcpy(h_packed, packed, packed_len * sizeof(float));
  if (use_graph) {
    if (!gexec_io) capture_io();
    CK_HIP(hipGraphLaunch(gexec_io, stream));
  } else {
    CK_HIP(hipMemcpyAsync(ptr("warped"), h_warped, warped_bytes, hipMemcpyHostToDevice, stream));
    CK_HIP(hipMemcpyAsync(ptr("packed"), h_packed, packed_len * sizeof(float), hipMemcpyHostToDevice, stream));
    launch_plan();
    CK_HIP(hipMemcpyAsync(h_out, ptr("out"), n_out * sizeof(float), hipMemcpyDeviceToHost, stream));
  }
  CK_HIP(hipStreamSynchronize(stream));
  std::memcpy(out, h_out, n_out * sizeof(float));
}

// The openpilot per-frame flow: two NV12 camera frames and their inverse
// transforms are staged, warped into `warped` on device (warp.hip), then the
// frame plan runs as in run_frame.  The warp is one launch ahead of the
// frame's graph.
void ck_engine::run_frame_nv12(const uint8_t* frame, const uint8_t* big_frame, const float* tfm, const float* big_tfm,
                               const float* packed, float* out) {
  CK_REQUIRE(nv12_bytes, "run_frame_nv12: the spec has no camera");
  uint8_t* nv = static_cast<uint8_t*>(ptr("nv12"));
  float* tf = static_cast<float*>(ptr("tfm"));
  // The two camera frames (3.7 MB each) go up in 2 MiB chunks: the copy into
  // the pinned staging of chunk k+1 overlaps the DMA of chunk k.  Two frames
  // staged whole and then copied take 232-236 us, in 2 MiB chunks 195 us (1
  // MiB: 221 us, 256 KiB: 390 us -- each copy call costs about 15-20 us);
  // the DMA alone is 139 us (54 GB/s).
  constexpr size_t CHUNK = size_t(2) << 20;
  for (int f = 0; f < 2; ++f) {
    const uint8_t* src = f == 0 ? frame : big_frame;
    for (size_t o = 0; o < nv12_bytes; o += CHUNK) {
      const size_t n = std::min(CHUNK, nv12_bytes - o);
      std::memcpy(h_nv12 + f * nv12_bytes + o, src + o, n);
      CK_HIP(hipMemcpyAsync(nv + f * nv12_bytes + o, h_nv12 + f * nv12_bytes + o, n, hipMemcpyHostToDevice, stream));
    }
  }
  std::memcpy(h_tfm, tfm, 9 * sizeof(float));
  std::memcpy(h_tfm + 9, big_tfm, 9 * sizeof(float));
  std::memcpy(h_packed, packed, packed_len * sizeof(float));
  CK_HIP(hipMemcpyAsync(tf, h_tfm, 18 * sizeof(float), hipMemcpyHostToDevice, stream));
  CK_HIP(hipMemcpyAsync(ptr("packed"), h_packed, packed_len * sizeof(float), hipMemcpyHostToDevice, stream));
  launch_warp_nv12(nv, nv + nv12_bytes, nv12_bytes, tf, tf + 9, sp.cam_w, sp.cam_h, sp.cam_stride, sp.cam_y_height,
                   2 * sp.img_w, 2 * sp.img_h, sp.cam_div, static_cast<uint8_t*>(ptr("warped")), stream);
  frame_launch();
  CK_HIP(hipMemcpyAsync(h_out, ptr("out"), n_out * sizeof(float), hipMemcpyDeviceToHost, stream));
  CK_HIP(hipStreamSynchronize(stream));
  std::memcpy(out, h_out, n_out * sizeof(float));
}

void ck_engine::reset_state() {
  for (const char* n : {"counter", "img_ring", "feat_ring", "desire_ring"}) {
    Tensor& t = tensor(n);
    launch_fill_u32(t.ptr, 0u, round_up((long)t.nbytes, 4) / 4, stream);
  }
  CK_HIP(hipStreamSynchronize(stream));
}

void ck_engine::run_range(int first, int last) {
  CK_REQUIRE(first >= 0 && last <= (int)plan.size() && first <= last, "run_range: bad plan range");
  for (int i = first; i < last; ++i) plan[i].fn(stream);
  CK_HIP(hipStreamSynchronize(stream));
}

void ck_engine::state_hashes(uint64_t* out, int n) {
  std::vector<const Tensor*> st;
  for (const auto& t : tensors)
    if (!t.param) st.push_back(&t);
  CK_REQUIRE(n >= (int)st.size(), "state_hashes: output array shorter than the state tensor count");
  if (!hash_part_dev) {
    for (int i = 0; i < (int)st.size(); ++i)
      for (size_t off = 0; off < st[i]->nbytes; off += HASH_SPAN_BYTES)
        hash_spans.push_back({static_cast<const uint8_t*>(st[i]->ptr), (long)off,
                              (int)std::min<size_t>(HASH_SPAN_BYTES, st[i]->nbytes - off), i});
    CK_REQUIRE(!hash_spans.empty(), "state_hashes: no state bytes");
    CK_HIP(hipMalloc(&hash_spans_dev, hash_spans.size() * sizeof(HashSpan)));
    CK_HIP(hipMalloc(&hash_part_dev, hash_spans.size() * sizeof(unsigned long long)));
    CK_HIP(hipMemcpy(hash_spans_dev, hash_spans.data(), hash_spans.size() * sizeof(HashSpan),
                     hipMemcpyHostToDevice));
  }
  launch_state_hash(hash_spans_dev, (int)hash_spans.size(), hash_part_dev, stream);
  std::vector<unsigned long long> part(hash_spans.size());
  CK_HIP(hipMemcpyAsync(part.data(), hash_part_dev, part.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost,
                        stream));
  CK_HIP(hipStreamSynchronize(stream));
  for (int i = 0; i < (int)st.size(); ++i) out[i] = hash_mix(st[i]->nbytes);
  for (size_t k = 0; k < hash_spans.size(); ++k) out[hash_spans[k].tensor] += part[k];
}

void ck_engine::kernel_times(float* ms, int n) {
  CK_REQUIRE(n >= (int)plan.size(), "kernel_times: output array shorter than the plan");
  hipEvent_t e0, e1;
  CK_HIP(hipEventCreate(&e0));
  CK_HIP(hipEventCreate(&e1));
  try {
    CK_HIP(hipStreamSynchronize(stream));
    for (size_t i = 0; i < plan.size(); ++i) {
      CK_HIP(hipEventRecord(e0, stream));
      plan[i].fn(stream);
      CK_HIP(hipEventRecord(e1, stream));
      CK_HIP(hipEventSynchronize(e1));
      CK_HIP(hipEventElapsedTime(&ms[i], e0, e1));
    }
  } catch (...) {
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    throw;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

// Kernel time of plan entries inside whole frames: `frames` eager frames of
// the full plan run back to back with no synchronisation between launches,
// and the entries listed in idx are launched with start/stop events (each
// kernel's own dispatch timestamps, see LaunchTimer).  per_entry_ms[k] = the
// kernel time of entry idx[k] per frame (an entry with a split-K reduce
// counts both kernels); returns the mean over the listed entries.
float ck_engine::time_in_frames(const int* idx, int n, int frames, float* per_entry_ms) {
  CK_REQUIRE(n > 0 && frames > 0, "time_in_frames: n and frames must be positive");
  std::vector<char> timed(plan.size(), 0);
  for (int k = 0; k < n; ++k) {
    CK_REQUIRE(idx[k] >= 0 && idx[k] < (int)plan.size(), "time_in_frames: plan index out of range");
    timed[idx[k]] = 1;
  }
  std::vector<std::vector<std::pair<hipEvent_t, hipEvent_t>>> events(plan.size());
  auto destroy = [&]() {
    for (auto& v : events)
      for (auto& e : v) {
        if (e.first) (void)hipEventDestroy(e.first);
        if (e.second) (void)hipEventDestroy(e.second);
      }
  };
  float total = 0.f;
  try {
    CK_HIP(hipStreamSynchronize(stream));
    for (int f = 0; f < frames; ++f) launch_plan(&timed, &events);
    CK_HIP(hipStreamSynchronize(stream));
    if (side) CK_HIP(hipStreamSynchronize(side));
    for (int k = 0; k < n; ++k) {
      float sum = 0.f;
      for (auto& e : events[idx[k]]) {
        float ms = 0.f;
        CK_HIP(hipEventElapsedTime(&ms, e.first, e.second));
        sum += ms;
      }
      if (per_entry_ms) per_entry_ms[k] = sum / frames;
      total += sum / frames;
    }
  } catch (...) {
    destroy();
    throw;
  }
  destroy();
  return total / n;
}

float ck_engine::time_launches(const int* idx, int n, int reps) {
  for (int i = 0; i < n; ++i)
    CK_REQUIRE(idx[i] >= 0 && idx[i] < (int)plan.size(), "time_launches: plan index out of range");
  hipEvent_t e0, e1;
  CK_HIP(hipEventCreate(&e0));
  CK_HIP(hipEventCreate(&e1));
  float ms = 0.f;
  try {
    CK_HIP(hipStreamSynchronize(stream));
    CK_HIP(hipEventRecord(e0, stream));
    for (int r = 0; r < reps; ++r)
      for (int i = 0; i < n; ++i) plan[idx[i]].fn(stream);
    CK_HIP(hipEventRecord(e1, stream));
    CK_HIP(hipEventSynchronize(e1));
    CK_HIP(hipEventElapsedTime(&ms, e0, e1));
  } catch (...) {
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    throw;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return ms;
}
