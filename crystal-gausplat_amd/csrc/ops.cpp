// Op-level C ABI: one entry point per NN::GPUOps operation on the MASt3R path
// (src/nn/gpu_ops.cr) plus the passes the reference runs on the CPU between
// GPU calls. Each call validates shapes on the host before any launch.
#include <hip/hip_runtime.h>
#include <string.h>

#include <map>
#include <mutex>
#include <vector>

#include "../../include/gs_hip.h"
#include "internal.h"

using namespace gs;

namespace {

hipStream_t pick(void* stream) { return (hipStream_t)stream; }

// Library-owned scratch for weight re-layouts of the op-level entry points
// (one per process; calls that need it are serialised by the mutex).
std::mutex g_ws_mu;
void* g_ws = nullptr;
size_t g_ws_size = 0;

int workspace(size_t bytes, void** out) {
  if (bytes > g_ws_size) {
    if (g_ws) {
      GS_CHECK_HIP(hipDeviceSynchronize());
      GS_CHECK_HIP(hipFree(g_ws));
      g_ws = nullptr;
      g_ws_size = 0;
    }
    GS_CHECK_HIP(hipMalloc(&g_ws, bytes));
    g_ws_size = bytes;
  }
  *out = g_ws;
  return 0;
}

// RoPE tables [512][16] per base, uploaded once.
std::mutex g_rope_mu;
std::map<float, std::pair<float*, float*>> g_rope;
constexpr int kRopeMaxPos = 512;

int rope_tables(float base, const float** c, const float** s) {
  std::lock_guard<std::mutex> lk(g_rope_mu);
  auto it = g_rope.find(base);
  if (it == g_rope.end()) {
    std::vector<float> hc(kRopeMaxPos * 16), hs(kRopeMaxPos * 16);
    rope_table_host(kRopeMaxPos, base, hc.data(), hs.data());
    float* dc = nullptr;
    float* ds = nullptr;
    GS_CHECK_HIP(hipMalloc(&dc, hc.size() * sizeof(float)));
    GS_CHECK_HIP(hipMalloc(&ds, hs.size() * sizeof(float)));
    GS_CHECK_HIP(hipMemcpy(dc, hc.data(), hc.size() * sizeof(float), hipMemcpyHostToDevice));
    GS_CHECK_HIP(hipMemcpy(ds, hs.data(), hs.size() * sizeof(float), hipMemcpyHostToDevice));
    it = g_rope.emplace(base, std::make_pair(dc, ds)).first;
  }
  *c = it->second.first;
  *s = it->second.second;
  return 0;
}

// Block-count scratch of gs_hip_collect_points (grown on demand).
std::mutex g_cp_mu;
int64_t* g_cp = nullptr;
int64_t g_cp_n = 0;

GemmArgs blank_args() {
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  return a;
}

}  // namespace

extern "C" {

int32_t gs_hip_linear(const float* x, const float* w, const float* b, float* y, int64_t M,
                      int32_t K, int32_t N, int32_t w_layout, int32_t epilogue,
                      const float* residual, void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(w_layout == 0 || w_layout == 1, "linear: w_layout must be 0 or 1");
  GS_REQUIRE(M >= 0 && M <= INT32_MAX, "linear: M out of range");
  GS_REQUIRE((epilogue & ~(GS_EPI_GELU | GS_EPI_RESIDUAL | GS_EPI_RELU | GS_EPI_BF16 |
                          GS_EPI_F32X6)) == 0,
             "linear: unknown epilogue flag");
  const bool x6 = (epilogue & GS_EPI_F32X6) != 0;
  GS_REQUIRE(!x6 || (w_layout == 0 && !(epilogue & GS_EPI_BF16)),
             "linear: the bf16x6 variant needs w_layout 0 and excludes the bf16 variant");
  const bool bf16 = (epilogue & GS_EPI_BF16) != 0;
  GS_REQUIRE(!bf16 || w_layout == 0, "linear: the bf16 variant needs w_layout 0");
  GS_REQUIRE(!(epilogue & GS_EPI_RESIDUAL) || residual, "linear: residual flag without residual");
  GemmArgs a = blank_args();
  a.A = x;
  a.lda = K;
  a.B = w;
  a.ldb = w_layout == 0 ? K : N;
  a.C = y;
  a.ldc = N;
  a.bias = b;
  a.M = (int32_t)M;
  a.N = N;
  a.K = K;
  a.flags = (b ? EPI_BIAS : 0) | ((epilogue & GS_EPI_GELU) ? EPI_GELU : 0) |
            ((epilogue & GS_EPI_RELU) ? EPI_RELU : 0) |
            ((epilogue & GS_EPI_RESIDUAL) ? EPI_RES1 : 0);
  a.R1 = residual;
  a.ldr1 = N;
  hipStream_t s = pick(stream);
  std::unique_lock<std::mutex> lk(g_ws_mu, std::defer_lock);
  if (bf16) {
    lk.lock();
    void* ws = nullptr;
    int rc = workspace((size_t)N * K * 2, &ws);
    if (rc) return rc;
    rc = launch_f32_to_bf16(w, ws, (int64_t)N * K, s);
    if (rc) return rc;
    a.Bh = ws;
  }
  GemmBatch bt;
  bt.g[0] = a;
  bt.ngroups = 1;
  if (x6) bt.kernel = 3;
  int rc = launch_gemm(bt, A_PLAIN, w_layout == 0 ? B_NT : B_NN, false, s, bf16);
  if (rc == 0 && bf16) GS_CHECK_HIP(hipStreamSynchronize(s));  // workspace reuse
  return rc;
}

int32_t gs_hip_layernorm(const float* x, const float* gamma, const float* beta, float* y,
                         int64_t rows, int32_t D, float eps, void* stream) {
  if (ensure_device()) return -2;
  LnBatch bt;
  bt.g[0] = LnArgs{x, gamma, beta, y, rows, D, eps};
  bt.ngroups = 1;
  return launch_layernorm(bt, pick(stream));
}

int32_t gs_hip_attention(const float* q, const float* k, const float* v, float* o, int32_t B,
                         int32_t H, int32_t Nq, int32_t Nkv, int32_t head_dim, float scale,
                         int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh,
                         int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn, int64_t o_sb,
                         int64_t o_sh, int64_t o_sn, void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(head_dim == 64, "attention: head_dim must be 64");
  AttnBatch bt;
  bt.g[0] = AttnArgs{q,    k,    v,    o,    q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb,
                     v_sh, v_sn, o_sb, o_sh, o_sn, B,    H,    Nq,   Nkv,  scale};
  bt.ngroups = 1;
  return launch_attention(bt, pick(stream));
}

int32_t gs_hip_rope2d(float* t, int32_t B, int32_t N, int32_t H, int64_t ld, int32_t grid_w,
                      float base, void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(grid_w > 0 && N > 0 && (N + grid_w - 1) / grid_w <= kRopeMaxPos &&
                 grid_w <= kRopeMaxPos,
             "rope2d: grid too large");
  const float* c = nullptr;
  const float* s = nullptr;
  int rc = rope_tables(base, &c, &s);
  if (rc) return rc;
  return launch_rope2d(t, B, N, H, ld, grid_w, c, s, pick(stream));
}

int32_t gs_hip_conv2d(const float* x, int32_t B, int32_t H, int32_t W, int32_t Cin,
                      const float* w, const float* b, float* y, int32_t Cout, int32_t k,
                      int32_t stride, int32_t pad, int32_t w_layout, int32_t flags,
                      const float* residual, void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(w_layout == 0 || w_layout == 1, "conv2d: w_layout must be 0 or 1");
  GS_REQUIRE(k > 0 && stride > 0 && pad >= 0 && B >= 0 && H > 0 && W > 0 && Cout > 0,
             "conv2d: bad geometry");
  GS_REQUIRE((flags & ~(GS_CONV_RELU_IN | GS_CONV_RELU_OUT | GS_CONV_F32X6)) == 0,
             "conv2d: unknown flag");
  const int32_t Ho = (H + 2 * pad - k) / stride + 1, Wo = (W + 2 * pad - k) / stride + 1;
  GS_REQUIRE(Ho > 0 && Wo > 0, "conv2d: empty output");
  GS_REQUIRE((int64_t)B * Ho * Wo <= INT32_MAX, "conv2d: too many output pixels");
  hipStream_t s = pick(stream);
  std::unique_lock<std::mutex> lk(g_ws_mu);
  const float* wk = w;
  if (w_layout == 0 && k > 1) {
    void* ws = nullptr;
    int rc = workspace((size_t)Cout * Cin * k * k * sizeof(float), &ws);
    if (rc) return rc;
    rc = launch_oihw_to_ohwi(w, Cout, Cin, k, (float*)ws, s);
    if (rc) return rc;
    wk = (const float*)ws;
  }
  GemmArgs a = blank_args();
  const bool pointwise = (k == 1 && stride == 1 && pad == 0);
  a.A = x;
  a.lda = Cin;
  a.cH = H;
  a.cW = W;
  a.cCin = Cin;
  a.ck = k;
  a.cs = stride;
  a.cp = pad;
  a.cHo = Ho;
  a.cWo = Wo;
  a.B = wk;
  a.ldb = (int64_t)k * k * Cin;
  a.C = y;
  a.ldc = Cout;
  a.bias = b;
  a.R1 = residual;
  a.ldr1 = Cout;
  a.M = (int32_t)((int64_t)B * Ho * Wo);
  a.N = Cout;
  a.K = k * k * Cin;
  a.flags = (b ? EPI_BIAS : 0) | ((flags & GS_CONV_RELU_OUT) ? EPI_RELU : 0) |
            (residual ? EPI_RES1 : 0);
  GemmBatch bt;
  bt.g[0] = a;
  bt.ngroups = 1;
  if (flags & GS_CONV_F32X6) bt.kernel = 3;
  int rc = launch_gemm(bt, pointwise ? A_PLAIN : A_CONV, B_NT, (flags & GS_CONV_RELU_IN) != 0, s);
  if (rc == 0 && wk != w) GS_CHECK_HIP(hipStreamSynchronize(s));  // workspace reuse
  return rc;
}

int32_t gs_hip_conv_transpose(const float* x, int32_t B, int32_t H, int32_t W, int32_t Cin,
                              const float* w, const float* b, float* y, int32_t Cout, int32_t k,
                              void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(k > 0 && Cin % 32 == 0 && Cout % 32 == 0 && B >= 0 && H > 0 && W > 0,
             "conv_transpose: need Cin % 32 == 0 and Cout % 32 == 0");
  GS_REQUIRE((int64_t)B * H * W <= INT32_MAX && (int64_t)k * k * Cout <= INT32_MAX,
             "conv_transpose: too many pixels");
  hipStream_t s = pick(stream);
  std::unique_lock<std::mutex> lk(g_ws_mu);
  const int64_t N = (int64_t)k * k * Cout;
  void* ws = nullptr;
  int rc = workspace((size_t)(N * Cin + N) * sizeof(float), &ws);
  if (rc) return rc;
  float* wt = (float*)ws;
  float* bt_exp = wt + N * Cin;
  rc = launch_convt_relayout(w, b, Cin, Cout, k, wt, bt_exp, s);
  if (rc) return rc;
  GemmArgs a = blank_args();
  a.A = x;
  a.lda = Cin;
  a.B = wt;
  a.ldb = Cin;
  a.C = y;
  a.ldc = N;
  a.bias = bt_exp;
  a.M = (int32_t)((int64_t)B * H * W);
  a.N = (int32_t)N;
  a.K = Cin;
  a.flags = EPI_BIAS | EPI_SCATTER;
  a.sc_r = k;
  a.sc_C = Cout;
  a.sc_Cout = Cout;
  a.sc_gh = H;
  a.sc_gw = W;
  GemmBatch bt;
  bt.g[0] = a;
  bt.ngroups = 1;
  rc = launch_gemm(bt, A_PLAIN, B_NT, false, s);
  if (rc == 0) GS_CHECK_HIP(hipStreamSynchronize(s));  // workspace reuse
  return rc;
}

int32_t gs_hip_upsample2x(const float* x, int32_t B, int32_t H, int32_t W, int32_t C, float* y,
                          void* stream) {
  if (ensure_device()) return -2;
  return launch_upsample2x(x, B, H, W, C, y, pick(stream));
}

int32_t gs_hip_resize_image(const float* src, int32_t F, int32_t sh, int32_t sw, int32_t C,
                            int32_t th, int32_t tw, float* dst, void* stream) {
  if (ensure_device()) return -2;
  return launch_image_prep(src, F, sh, sw, C, th, tw, true, false, false, dst, pick(stream));
}

int32_t gs_hip_preprocess_image(const float* src, int32_t B, int32_t H, int32_t W, float* dst,
                                void* stream) {
  if (ensure_device()) return -2;
  return launch_image_prep(src, B, H, W, 3, H, W, false, true, true, dst, pick(stream));
}

int32_t gs_hip_prepare_frames(const float* src, int32_t F, int32_t sh, int32_t sw, int32_t th,
                              int32_t tw, float* dst, void* stream) {
  if (ensure_device()) return -2;
  return launch_image_prep(src, F, sh, sw, 3, th, tw, true, true, true, dst, pick(stream));
}

int32_t gs_hip_collect_points(const float* pts, const float* conf, int64_t n, float threshold,
                              float* out_pts, float* out_conf, int64_t capacity, int64_t* count,
                              void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(n >= 0, "collect_points: n < 0");
  std::lock_guard<std::mutex> lk(g_cp_mu);
  const int64_t need = collect_points_scratch(n);
  if (need > g_cp_n) {
    if (g_cp) {
      GS_CHECK_HIP(hipDeviceSynchronize());
      GS_CHECK_HIP(hipFree(g_cp));
      g_cp = nullptr;
      g_cp_n = 0;
    }
    GS_CHECK_HIP(hipMalloc(&g_cp, need * sizeof(int64_t)));
    g_cp_n = need;
  }
  return launch_collect_points(pts, conf, n, threshold, out_pts, out_conf, capacity, count, g_cp,
                               pick(stream));
}

}  // extern "C"
