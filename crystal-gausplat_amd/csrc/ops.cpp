// Op-level C ABI: one entry point per NN::GPUOps operation on the MASt3R path
// (src/nn/gpu_ops.cr) plus the passes the reference runs on the CPU between
// GPU calls. Each call validates shapes on the host before any launch.
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <vector>

#include "../../include/gs_hip.h"
#include "internal.h"

using namespace gs;

namespace {

hipStream_t pick(void* stream) { return (hipStream_t)stream; }

// Scratch of one op-level call (weight re-layouts, zero-padded operand copies,
// compaction block counts): allocated on the call's stream and released on it
// after the kernels that use it (stream-ordered allocation). Calls on
// different streams never share scratch and no call waits for the device.
class StreamScratch {
 public:
  ~StreamScratch() {
    if (p_) (void)hipFreeAsync(p_, s_);
  }
  int alloc(size_t bytes, hipStream_t s) {
    s_ = s;
    GS_CHECK_HIP(hipMallocAsync(&p_, bytes ? bytes : 16, s));
    return 0;
  }
  char* get() const { return (char*)p_; }

 private:
  void* p_ = nullptr;
  hipStream_t s_ = nullptr;
};

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Split-K / key-split partials of an op-level call whose launch would leave
// most CUs idle (fewer than ~432 workgroups): up to 16 partial tiles per
// output, capped at 64 MB (the launchers pick a smaller split that fits).
// A split keeps at least 4 K steps of 32 per range, so K below 256 never
// splits and reserves nothing.
constexpr int64_t kOpSplitCapBytes = (int64_t)64 << 20;
int64_t gemm_split_bytes(int64_t M, int64_t N, int64_t K, int ngroups = 1) {
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128) * ngroups;
  if (tiles >= 432 || K / 32 < 8) return 0;
  return std::min<int64_t>(16 * M * N * 4 * ngroups, kOpSplitCapBytes);
}

// RoPE tables [512][16] per (device, base), uploaded once per device.
std::mutex g_rope_mu;
std::map<std::pair<int, float>, std::pair<float*, float*>> g_rope;
constexpr int kRopeMaxPos = 512;

int rope_tables(float base, const float** c, const float** s) {
  int dev = 0;
  GS_CHECK_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_rope_mu);
  const std::pair<int, float> key(dev, base);
  auto it = g_rope.find(key);
  if (it == g_rope.end()) {
    std::vector<float> hc(kRopeMaxPos * 16), hs(kRopeMaxPos * 16);
    rope_table_host(kRopeMaxPos, base, hc.data(), hs.data());
    float* dc = nullptr;
    float* ds = nullptr;
    GS_CHECK_HIP(hipMalloc(&dc, hc.size() * sizeof(float)));
    GS_CHECK_HIP(hipMalloc(&ds, hs.size() * sizeof(float)));
    GS_CHECK_HIP(hipMemcpy(dc, hc.data(), hc.size() * sizeof(float), hipMemcpyHostToDevice));
    GS_CHECK_HIP(hipMemcpy(ds, hs.data(), hs.size() * sizeof(float), hipMemcpyHostToDevice));
    it = g_rope.emplace(key, std::make_pair(dc, ds)).first;
  }
  *c = it->second.first;
  *s = it->second.second;
  return 0;
}

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
  GS_REQUIRE(K > 0 && N > 0, "linear: K and N must be positive");
  GS_REQUIRE(x && w && y, "linear: null operand");
  GS_REQUIRE((epilogue & ~(GS_EPI_GELU | GS_EPI_RESIDUAL | GS_EPI_RELU | GS_EPI_BF16 |
                          GS_EPI_F32X6)) == 0,
             "linear: unknown epilogue flag");
  const bool x6 = (epilogue & GS_EPI_F32X6) != 0;
  GS_REQUIRE(!x6 || (w_layout == 0 && !(epilogue & GS_EPI_BF16)),
             "linear: the bf16x6 variant needs w_layout 0 and excludes the bf16 variant");
  const bool bf16 = (epilogue & GS_EPI_BF16) != 0;
  GS_REQUIRE(!bf16 || w_layout == 0, "linear: the bf16 variant needs w_layout 0");
  GS_REQUIRE(!(epilogue & GS_EPI_RESIDUAL) || residual, "linear: residual flag without residual");
  if (M == 0) return 0;
  hipStream_t s = pick(stream);
  // The MFMA GEMM takes K in steps of 32 from 16-byte aligned rows. Other
  // shapes (the reference's linear_forward takes any width) run on
  // zero-padded copies: x -> [M, Kp], W -> [N, Kp] (NT, either layout); the
  // padded products are exact zeros, so the sums are those of the K terms.
  const bool kfit = K % 32 == 0;
  const bool stage_a = !kfit || !aligned16(x);
  const bool stage_b = !kfit || !aligned16(w) || (w_layout == 1 && N % 4 != 0);
  const int64_t Kp = round_up(K, 32);
  // scratch: [staged x | staged W | bf16 copy of W | bf16 copy of x], each
  // part 256-byte aligned. The bf16 variant reads bf16 activations (the
  // A_PLAIN_H loader): x is rounded once here, with the round-to-nearest-even
  // the fp32-row loader applies, so the products are the same.
  const int64_t a_bytes = stage_a ? M * Kp * 4 : 0;
  const int64_t b_bytes = stage_b ? (int64_t)N * Kp * 4 : 0;
  const int64_t h_bytes = bf16 ? (int64_t)N * Kp * 2 : 0;
  const int64_t xh_bytes = bf16 ? M * Kp * 2 : 0;
  const int64_t off_b = round_up(a_bytes, 256), off_h = round_up(off_b + b_bytes, 256);
  const int64_t off_xh = round_up(off_h + h_bytes, 256);
  const int64_t off_p = round_up(off_xh + xh_bytes, 256), p_bytes = gemm_split_bytes(M, N, Kp);
  StreamScratch ws;
  if (off_p + p_bytes > 0) {
    int rc = ws.alloc((size_t)(off_p + p_bytes), s);
    if (rc) return rc;
  }
  const float* A = x;
  const float* Bw = w;
  int64_t lda = K, ldb = w_layout == 0 ? K : N;
  int blayout = w_layout == 0 ? B_NT : B_NN;
  if (stage_a) {
    float* as = (float*)ws.get();
    int rc = launch_stage(x, M, K, K, 1, as, Kp, s);
    if (rc) return rc;
    A = as;
    lda = Kp;
  }
  if (stage_b) {
    float* bs = (float*)(ws.get() + off_b);
    int rc = w_layout == 0 ? launch_stage(w, N, K, K, 1, bs, Kp, s)
                           : launch_stage(w, N, K, 1, N, bs, Kp, s);
    if (rc) return rc;
    Bw = bs;
    ldb = Kp;
    blayout = B_NT;
  }
  GemmArgs a = blank_args();
  a.A = A;
  a.lda = lda;
  a.B = Bw;
  a.ldb = ldb;
  a.C = y;
  a.ldc = N;
  a.bias = b;
  a.M = (int32_t)M;
  a.N = N;
  a.K = kfit ? K : (int32_t)Kp;
  a.flags = (b ? EPI_BIAS : 0) | ((epilogue & GS_EPI_GELU) ? EPI_GELU : 0) |
            ((epilogue & GS_EPI_RELU) ? EPI_RELU : 0) |
            ((epilogue & GS_EPI_RESIDUAL) ? EPI_RES1 : 0);
  a.R1 = residual;
  a.ldr1 = N;
  if (bf16) {
    void* wh = ws.get() + off_h;
    int rc = launch_f32_to_bf16(Bw, wh, (int64_t)N * a.ldb, s);
    if (rc) return rc;
    a.Bh = wh;
    void* xh = ws.get() + off_xh;
    rc = launch_f32_to_bf16(A, xh, M * lda, s);
    if (rc) return rc;
    a.A = (const float*)xh;  // bf16 rows, lda elements apart
  }
  GemmBatch bt;
  bt.g[0] = a;
  bt.ngroups = 1;
  if (x6) bt.kernel = 3;
  if (p_bytes) {
    bt.part_ws = (float*)(ws.get() + off_p);
    bt.part_ws_elems = p_bytes / 4;
  }
  return launch_gemm(bt, bf16 ? A_PLAIN_H : A_PLAIN, blayout, false, s, bf16);
}

int32_t gs_hip_layernorm(const float* x, const float* gamma, const float* beta, float* y,
                         int64_t rows, int32_t D, float eps, void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(D > 0 && rows >= 0, "layernorm: bad sizes");
  const LnArgs a{x, gamma, beta, y, rows, D, eps};
  // one wavefront per row for aligned rows of D % 4 == 0 up to 4096, one
  // workgroup per row (any width and alignment) otherwise
  if (D % 4 == 0 && D <= 4096 && aligned16(x) && aligned16(y) && aligned16(gamma) &&
      aligned16(beta)) {
    LnBatch bt;
    bt.g[0] = a;
    bt.ngroups = 1;
    return launch_layernorm(bt, pick(stream));
  }
  return launch_layernorm_rows(a, pick(stream));
}

int32_t gs_hip_attention_prec(const float* q, const float* k, const float* v, float* o,
                              int32_t B, int32_t H, int32_t Nq, int32_t Nkv, int32_t head_dim,
                              float scale, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb,
                              int64_t k_sh, int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn,
                              int64_t o_sb, int64_t o_sh, int64_t o_sn, int32_t precision,
                              void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(head_dim >= 1, "attention: head_dim must be >= 1");
  GS_REQUIRE(precision >= 0 && precision <= 2, "attention: precision must be 0, 1 or 2");
  const AttnArgs a{q,    k,    v,    o,    q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb,
                   v_sh, v_sn, o_sb, o_sh, o_sn, B,    H,    Nq,   Nkv,  scale};
  // head_dim 64 with 16-byte aligned rows runs on the MFMA flash kernels;
  // other head dims and layouts on the general fp32 kernel (one wavefront per
  // query), which the bf16 variants do not have
  bool mfma = head_dim == 64 && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
  const int64_t st[12] = {q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn, o_sb, o_sh, o_sn};
  for (int j = 0; j < 12; ++j) mfma = mfma && st[j] % 4 == 0;
  // the MFMA kernels' buffer-resource K / V loads: key rows at least 64
  // floats apart, each (image, head) K / V span below 2 GiB
  mfma = mfma && k_sn >= 64 && v_sn >= 64 && Nkv > 0 &&
         ((int64_t)(Nkv - 1) * std::max(k_sn, v_sn) + 64) * 4 < ((int64_t)1 << 31);
  GS_REQUIRE(mfma || precision == 0,
             "attention: the bf16 and bf16x6 variants need head_dim 64 and 16-byte aligned rows "
             "(pointers and strides multiples of 4 floats)");
  if (!mfma) return launch_attention_general(a, head_dim, pick(stream));
  AttnBatch bt;
  bt.g[0] = a;
  bt.ngroups = 1;
  // launches that leave most CUs idle split the keys into ranges merged in
  // order; their partial states live in stream-ordered scratch sized by the
  // launcher's own rule (zero when this launch cannot split)
  StreamScratch ws;
  const int64_t elems = std::min<int64_t>(attention_split_elems(bt, precision), kOpSplitCapBytes / 4) / 4 * 4;
  if (elems > 0) {
    int rc = ws.alloc((size_t)elems * 4, pick(stream));
    if (rc) return rc;
    bt.part_ws = (float*)ws.get();
    bt.part_ws_elems = elems;
  }
  return launch_attention(bt, pick(stream), precision);
}

int32_t gs_hip_attention(const float* q, const float* k, const float* v, float* o, int32_t B,
                         int32_t H, int32_t Nq, int32_t Nkv, int32_t head_dim, float scale,
                         int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh,
                         int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn, int64_t o_sb,
                         int64_t o_sh, int64_t o_sn, void* stream) {
  return gs_hip_attention_prec(q, k, v, o, B, H, Nq, Nkv, head_dim, scale, q_sb, q_sh, q_sn, k_sb,
                               k_sh, k_sn, v_sb, v_sh, v_sn, o_sb, o_sh, o_sn, 0, stream);
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

int32_t gs_hip_conv2d_hw(const float* x, int32_t B, int32_t H, int32_t W, int32_t Cin,
                         const float* w, const float* b, float* y, int32_t Cout, int32_t kh,
                         int32_t kw, int32_t stride, int32_t pad, int32_t w_layout, int32_t flags,
                         const float* residual, void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(w_layout == 0 || w_layout == 1, "conv2d: w_layout must be 0 or 1");
  GS_REQUIRE(kh > 0 && kw > 0 && stride > 0 && pad >= 0 && B >= 0 && H > 0 && W > 0 && Cin > 0 &&
                 Cout > 0,
             "conv2d: bad geometry");
  GS_REQUIRE(x && w && y, "conv2d: null operand");
  GS_REQUIRE((flags & ~(GS_CONV_RELU_IN | GS_CONV_RELU_OUT | GS_CONV_F32X6)) == 0,
             "conv2d: unknown flag");
  GS_REQUIRE(H + 2 * pad >= kh && W + 2 * pad >= kw, "conv2d: empty output");
  const int32_t Ho = (H + 2 * pad - kh) / stride + 1, Wo = (W + 2 * pad - kw) / stride + 1;
  GS_REQUIRE((int64_t)B * Ho * Wo <= INT32_MAX, "conv2d: too many output pixels");
  GS_REQUIRE((int64_t)B * H * W <= INT32_MAX, "conv2d: too many input pixels");
  if (B == 0) return 0;
  hipStream_t s = pick(stream);
  // The implicit-GEMM conv reads 32 input channels per K step from 16-byte
  // aligned NHWC rows, with the weight as OHWI. An OIHW weight is re-laid
  // per call (the caller keeps ownership; a weight may change between calls);
  // other channel counts run on copies zero-padded to a multiple of 32.
  const int32_t Cp = (int32_t)round_up(Cin, 32);
  const bool stage_x = Cp != Cin || !aligned16(x);
  const bool stage_w = Cp != Cin || !aligned16(w) || (w_layout == 0 && kh * kw > 1);
  const int64_t x_bytes = stage_x ? (int64_t)B * H * W * Cp * 4 : 0;
  const int64_t w_bytes = stage_w ? (int64_t)Cout * kh * kw * Cp * 4 : 0;
  const int64_t off_w = round_up(x_bytes, 256), off_p = round_up(off_w + w_bytes, 256);
  const int64_t p_bytes = gemm_split_bytes((int64_t)B * Ho * Wo, Cout, (int64_t)kh * kw * Cp);
  StreamScratch ws;
  if (off_p + p_bytes > 0) {
    int rc = ws.alloc((size_t)(off_p + p_bytes), s);
    if (rc) return rc;
  }
  const float* xk = x;
  const float* wk = w;
  if (stage_x) {
    float* xs = (float*)ws.get();
    int rc = launch_stage(x, (int64_t)B * H * W, Cin, Cin, 1, xs, Cp, s);
    if (rc) return rc;
    xk = xs;
  }
  if (stage_w) {
    float* wsb = (float*)(ws.get() + off_w);
    int rc = launch_conv_weight_stage(w, Cout, Cin, kh, kw, w_layout, Cp, wsb, s);
    if (rc) return rc;
    wk = wsb;
  }
  GemmArgs a = blank_args();
  const bool pointwise = (kh == 1 && kw == 1 && stride == 1 && pad == 0);
  a.A = xk;
  a.lda = Cp;
  a.cH = H;
  a.cW = W;
  a.cCin = Cp;
  a.ck = kh;
  a.ckw = kw;
  a.cs = stride;
  a.cp = pad;
  a.cHo = Ho;
  a.cWo = Wo;
  a.B = wk;
  a.ldb = (int64_t)kh * kw * Cp;
  a.C = y;
  a.ldc = Cout;
  a.bias = b;
  a.R1 = residual;
  a.ldr1 = Cout;
  a.M = (int32_t)((int64_t)B * Ho * Wo);
  a.N = Cout;
  a.K = kh * kw * Cp;
  a.flags = (b ? EPI_BIAS : 0) | ((flags & GS_CONV_RELU_OUT) ? EPI_RELU : 0) |
            (residual ? EPI_RES1 : 0);
  GemmBatch bt;
  bt.g[0] = a;
  bt.ngroups = 1;
  if (flags & GS_CONV_F32X6) bt.kernel = 3;
  if (p_bytes) {
    bt.part_ws = (float*)(ws.get() + off_p);
    bt.part_ws_elems = p_bytes / 4;
  }
  return launch_gemm(bt, pointwise ? A_PLAIN : A_CONV, B_NT, (flags & GS_CONV_RELU_IN) != 0, s);
}

int32_t gs_hip_conv2d(const float* x, int32_t B, int32_t H, int32_t W, int32_t Cin,
                      const float* w, const float* b, float* y, int32_t Cout, int32_t k,
                      int32_t stride, int32_t pad, int32_t w_layout, int32_t flags,
                      const float* residual, void* stream) {
  return gs_hip_conv2d_hw(x, B, H, W, Cin, w, b, y, Cout, k, k, stride, pad, w_layout, flags,
                          residual, stream);
}

int32_t gs_hip_conv_transpose(const float* x, int32_t B, int32_t H, int32_t W, int32_t Cin,
                              const float* w, const float* b, float* y, int32_t Cout, int32_t k,
                              void* stream) {
  if (ensure_device()) return -2;
  GS_REQUIRE(k > 0 && Cin % 32 == 0 && Cout % 32 == 0 && B >= 0 && H > 0 && W > 0,
             "conv_transpose: need Cin % 32 == 0 and Cout % 32 == 0");
  GS_REQUIRE((int64_t)B * H * W <= INT32_MAX && (int64_t)k * k * Cout <= INT32_MAX,
             "conv_transpose: too many pixels");
  GS_REQUIRE(x && w && y, "conv_transpose: null operand");
  if (B == 0) return 0;
  hipStream_t s = pick(stream);
  const int64_t N = (int64_t)k * k * Cout;
  StreamScratch ws;
  int rc = ws.alloc((size_t)(N * Cin + N) * sizeof(float), s);
  if (rc) return rc;
  float* wt = (float*)ws.get();
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
  return launch_gemm(bt, A_PLAIN, B_NT, false, s);
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
  if (n == 0) return launch_collect_points(pts, conf, 0, threshold, out_pts, out_conf, capacity,
                                           count, nullptr, pick(stream));
  hipStream_t s = pick(stream);
  StreamScratch ws;
  int rc = ws.alloc((size_t)collect_points_scratch(n) * sizeof(int64_t), s);
  if (rc) return rc;
  return launch_collect_points(pts, conf, n, threshold, out_pts, out_conf, capacity, count,
                               (int64_t*)ws.get(), s);
}

}  // extern "C"
