// MASt3R two-view inference on one GPU: the graph-level entry points.
//
// Host-side mirror of the reference model classes (same roles, same order of
// operations) driving the gfx950 kernels as one launch sequence on a stream:
//   MASt3REncoderV2 / MASt3REncoderBlockV2   src/mastr/encoder_v2.cr:15-259
//   MASt3RDecoder / MASt3RDecoderBlock       src/mastr/decoder_v2.cr:16-201
//   DPTHead / RefineNetBlock / RCU           src/mastr/decoder_v2.cr:356-656
//   MASt3RInference#forward_pair             src/mastr/inference.cr:92-115
// Differences from the reference's literal composition follow the MASt3R
// configuration (per-attention 2D RoPE, cross-attention to the other view,
// full DPT, 1+exp confidence, local-feature descriptors).
//
// Data layout in HBM: tokens are row-major [rows, dim] with the two views
// stacked (view 1 rows first), i.e. NHWC on the patch grid; DPT activations
// are NHWC; weights are stored once per context in one arena, linears as
// [out, in], 3x3 convs re-laid to [out, kh, kw, in] (K contiguous for the
// implicit GEMM), ConvTranspose to [(i*k+j)*out + oc, in], the cross-attention
// k/v projections concatenated to one [2D, D] weight, and the descriptor MLP's
// second layer permuted so its GEMM columns are (sub-pixel, channel) pairs of
// the 24 kept channels.
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "../../include/gs_hip.h"
#include "internal.h"

using namespace gs;

namespace {

// ---------------------------------------------------------------------------
// Weight inventory (checkpoint naming, src/mastr/weight_loader.cr:43-123)
// ---------------------------------------------------------------------------
enum WKind { W_WEIGHT = 0, W_BIAS = 1, W_GAMMA = 2, W_BETA = 3 };
// How a host tensor is placed on the device.
enum Place {
  P_PLAIN = 0,    // copied as is
  P_CONV = 1,     // OIHW -> OHWI
  P_CONVT_W = 2,  // [Cin,Cout,k,k] -> [(i*k+j)*Cout+oc][Cin]
  P_CONVT_B = 3,  // bias expanded to k*k*Cout
  P_KV = 4,       // rows [off, off+rows) of the concatenated k|v weight/bias
  P_DESC_W = 5,   // descriptor fc2 rows permuted, channel >= desc dropped
  P_DESC_B = 6,
};

struct WInfo {
  std::string name;
  int64_t shape[4];
  int kind;
};

struct Inventory {
  std::vector<WInfo> w;
  void add(const std::string& n, std::initializer_list<int64_t> s, int kind) {
    WInfo x;
    x.name = n;
    int i = 0;
    for (int64_t v : s) x.shape[i++] = v;
    for (; i < 4; ++i) x.shape[i] = 0;
    x.kind = kind;
    w.push_back(x);
  }
  void linear(const std::string& n, int64_t out, int64_t in, bool bias = true) {
    add(n + ".weight", {out, in}, W_WEIGHT);
    if (bias) add(n + ".bias", {out}, W_BIAS);
  }
  void conv(const std::string& n, int64_t out, int64_t in, int64_t k, bool bias = true) {
    add(n + ".weight", {out, in, k, k}, W_WEIGHT);
    if (bias) add(n + ".bias", {out}, W_BIAS);
  }
  void norm(const std::string& n, int64_t d) {
    add(n + ".weight", {d}, W_GAMMA);
    add(n + ".bias", {d}, W_BETA);
  }
};

Inventory make_inventory(const gs_mastr_config& c) {
  Inventory v;
  const int64_t De = c.enc_dim, Dd = c.dec_dim, F = c.dpt_feat;
  v.conv("patch_embed.proj", De, 3, c.patch);
  for (int l = 0; l < c.enc_depth; ++l) {
    const std::string p = "enc_blocks." + std::to_string(l);
    v.norm(p + ".norm1", De);
    v.linear(p + ".attn.qkv", 3 * De, De);
    v.linear(p + ".attn.proj", De, De);
    v.norm(p + ".norm2", De);
    v.linear(p + ".mlp.fc1", c.enc_mlp, De);
    v.linear(p + ".mlp.fc2", De, c.enc_mlp);
  }
  v.norm("enc_norm", De);
  v.linear("decoder_embed", Dd, De);
  for (int chain = 0; chain < 2; ++chain)
    for (int l = 0; l < c.dec_depth; ++l) {
      const std::string p = (chain ? "dec_blocks2." : "dec_blocks.") + std::to_string(l);
      v.norm(p + ".norm1", Dd);
      v.linear(p + ".attn.qkv", 3 * Dd, Dd);
      v.linear(p + ".attn.proj", Dd, Dd);
      v.norm(p + ".norm2", Dd);
      v.norm(p + ".norm3", Dd);
      v.norm(p + ".norm_y", Dd);
      v.linear(p + ".cross_attn.projq", Dd, Dd);
      v.linear(p + ".cross_attn.projk", Dd, Dd);
      v.linear(p + ".cross_attn.projv", Dd, Dd);
      v.linear(p + ".cross_attn.proj", Dd, Dd);
      v.linear(p + ".mlp.fc1", c.dec_mlp, Dd);
      v.linear(p + ".mlp.fc2", Dd, c.dec_mlp);
    }
  v.norm("dec_norm", Dd);
  for (int hd = 1; hd <= 2; ++hd) {
    const std::string p = "downstream_head" + std::to_string(hd);
    const std::string ap = p + ".dpt.act_postprocess.";
    const int64_t d[4] = {c.dpt_dims[0], c.dpt_dims[1], c.dpt_dims[2], c.dpt_dims[3]};
    v.conv(ap + "0.0", d[0], De, 1);
    v.conv(ap + "0.1", d[0], d[0], 4);  // ConvTranspose [in, out, 4, 4]
    v.conv(ap + "1.0", d[1], Dd, 1);
    v.conv(ap + "1.1", d[1], d[1], 2);  // ConvTranspose [in, out, 2, 2]
    v.conv(ap + "2.0", d[2], Dd, 1);
    v.conv(ap + "3.0", d[3], Dd, 1);
    v.conv(ap + "3.1", d[3], d[3], 3);
    for (int i = 0; i < 4; ++i)
      v.conv(p + ".dpt.scratch.layer" + std::to_string(i + 1) + "_rn", F, d[i], 3, false);
    for (int r = 1; r <= 4; ++r) {
      const std::string rp = p + ".dpt.scratch.refinenet" + std::to_string(r);
      // refinenet4's first unit has no input in the full DPT (no skip at the
      // deepest level) but is in the checkpoint and in the reference's stub
      for (int u = 1; u <= 2; ++u) {
        v.conv(rp + ".resConfUnit" + std::to_string(u) + ".conv1", F, F, 3);
        v.conv(rp + ".resConfUnit" + std::to_string(u) + ".conv2", F, F, 3);
      }
      v.conv(rp + ".out_conv", F, F, 1);
    }
    v.conv(p + ".dpt.head.0", F / 2, F, 3);
    v.conv(p + ".dpt.head.2", c.head_mid, F / 2, 3);
    v.conv(p + ".dpt.head.4", 4, c.head_mid, 1);
    v.linear(p + ".head_local_features.fc1", c.lf_hidden, De + Dd);
    v.linear(p + ".head_local_features.fc2", (int64_t)(c.desc_dim + 1) * c.patch * c.patch,
             c.lf_hidden);
  }
  return v;
}

int64_t numel(const WInfo& w) {
  int64_t n = 1;
  for (int i = 0; i < 4 && w.shape[i]; ++i) n *= w.shape[i];
  return n;
}

// ---------------------------------------------------------------------------
// Context
// ---------------------------------------------------------------------------
struct DevW {
  float* ptr = nullptr;
  int place = P_PLAIN;
  int64_t host_numel = 0;
  int64_t a = 0, b = 0, c = 0, d = 0;  // placement parameters
};

struct Ctx {
  gs_mastr_config cfg;
  int max_pairs = 0;
  int gh = 0, gw = 0, N = 0;
  Inventory inv;
  std::map<std::string, DevW> w;
  std::map<std::string, float*> derived;  // kv weights etc. by name
  char* warena = nullptr;
  size_t warena_size = 0;
  char* wbf16 = nullptr;     // bf16 mirror of warena (precision 1), or its
                             // three-plane bf16 split (precision 2)
  bool bf16_dirty = true;
  char* arena = nullptr;
  size_t arena_size = 0;
  // workspaces
  float *P, *x, *h, *qkv, *att, *mlp, *enc, *d, *ym, *kv, *q, *hook1, *hook2, *dfin;
  float* lnst;  // (mean, inv_std) per row of the LayerNorms fused into GEMM loads
  float* dmem;  // composite 1: decoder_embed output, the fixed cross-attention memory
  float* splitk;  // split-K partial tiles of small GEMM launches (kSplitkElems floats)
  // DPT / descriptor workspaces, one slot per head of a grouped launch
  float *t0[2], *act[2][4], *L[2][4], *u[2], *s[2], *t[2], *up[2], *rA[2], *rB[2], *hd0[2],
      *hup[2], *hd2[2], *lf[2];
  float* Lh[2][4];  // bf16 mode: bf16(max(L, 0)), the inputs of the RCU conv1s that read L
  float *rope_cos, *rope_sin, *ref_cos, *ref_sin;
  int ref_maxpos = 0;
  int last_B = 0;
  // hipGraph replay of the pair launch sequence (gs_hip_mastr_set_graph)
  bool graph_on = false;
  hipGraphExec_t gexec = nullptr;
  const void* gkey[9] = {};
  int gkey_B = 0;
  // frames_to_pointcloud buffers (prepared frames, per-chunk point maps,
  // compaction counter and scratch), grown on demand
  char* pcbuf = nullptr;
  size_t pcbuf_size = 0;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Split-K scratch per context: 64 MB covers the partial tiles of every launch
// that leaves CUs idle at one pair (launch_gemm lowers the split otherwise).
constexpr int64_t kSplitkElems = (int64_t)16 << 20;

GemmArgs blank() {
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  return a;
}

GemmArgs lin(const float* A, int64_t lda, const float* W, const float* bias, float* C,
             int64_t ldc, int64_t M, int N, int K, int flags) {
  GemmArgs a = blank();
  a.A = A;
  a.lda = lda;
  a.B = W;
  a.ldb = K;
  a.C = C;
  a.ldc = ldc;
  a.bias = bias;
  a.M = (int32_t)M;
  a.N = N;
  a.K = K;
  a.flags = flags | (bias ? EPI_BIAS : 0);
  return a;
}

void with_rope(GemmArgs& a, const Ctx& c, int ncols) {
  a.flags |= EPI_ROPE;
  a.rope_cos = c.rope_cos;
  a.rope_sin = c.rope_sin;
  a.rope_ncols = ncols;
  a.tok_per_img = c.N;
  a.grid_w = c.gw;
}

// All context GEMMs go through here: in the bf16 precision mode each group's
// weight operand is redirected to its bf16 mirror.
int gemm(const Ctx& c, GemmBatch& b, int aload, bool relu_in, hipStream_t s) {
  const bool bf = c.cfg.precision == 1;
  if (bf)
    for (int i = 0; i < b.ngroups; ++i) {
      const char* w = (const char*)b.g[i].B;
      GS_REQUIRE(w >= c.warena && w < c.warena + c.warena_size, "gemm: weight outside the arena");
      b.g[i].Bh = c.wbf16 + (w - c.warena) / 2;
    }
  b.part_ws = c.splitk;
  b.part_ws_elems = kSplitkElems;
  if (c.cfg.precision == 2) {  // fp32 through bf16x6 split products, weights pre-split
    b.kernel = 3;
    for (int i = 0; i < b.ngroups; ++i) {
      const char* w = (const char*)b.g[i].B;
      GS_REQUIRE(w >= c.warena && w < c.warena + c.warena_size, "gemm: weight outside the arena");
      b.g[i].Bh = c.wbf16 + (w - c.warena) / 2;
      b.g[i].bh_plane = (int64_t)(c.warena_size / 4);
    }
  }
  return launch_gemm(b, aload, B_NT, relu_in, s, bf);
}

// All context attention launches go through here (scratch for key splits).
int attention(const Ctx& c, AttnBatch& ab, hipStream_t s) {
  ab.part_ws = c.splitk;
  ab.part_ws_elems = kSplitkElems;
  return launch_attention(ab, s, c.cfg.precision);
}

int run1(const Ctx& c, const GemmArgs& a, int aload, hipStream_t s, bool relu_in = false) {
  GemmBatch b;
  b.g[0] = a;
  b.ngroups = 1;
  return gemm(c, b, aload, relu_in, s);
}

int run2(const Ctx& c, const GemmArgs& a0, const GemmArgs& a1, int aload, hipStream_t s) {
  GemmBatch b;
  b.g[0] = a0;
  b.g[1] = a1;
  b.ngroups = 2;
  return gemm(c, b, aload, false, s);
}

#define RC(expr)              \
  do {                        \
    int rc_ = (expr);         \
    if (rc_) return rc_;      \
  } while (0)

const float* W(Ctx& c, const std::string& n) {
  auto it = c.w.find(n);
  return it == c.w.end() ? nullptr : it->second.ptr;
}

// Linear under the context's layout mode (D1). groups > 1 splits a fused
// weight into that many reference Linear modules for the literal layout.
// LayerNorm applied in the GEMM's A load (A_LN): row statistics, gamma, beta.
struct LnFuse {
  const float* stats = nullptr;
  const float* g = nullptr;
  const float* b = nullptr;
};

// The LayerNorm that follows a GEMM on its output rows (EPI_LNOUT): gamma,
// beta and the destination of the normalised rows.
struct LnNext {
  const float* g = nullptr;
  const float* b = nullptr;
  float* y = nullptr;
};

void with_lnout(GemmArgs& a, const Ctx& c, const LnNext& n) {
  a.flags |= EPI_LNOUT;
  a.lnout = n.y;
  a.lnout_g = n.g;
  a.lnout_b = n.b;
  a.lnout_eps = c.cfg.ln_eps;
}

int linear_mode(Ctx& c, const std::string& name, const float* A, int64_t lda, float* C,
                int64_t ldc, int64_t M, int N, int K, int flags, hipStream_t s, int groups = 1,
                int rope_cols = 0, int aload = A_PLAIN, LnFuse lnf = LnFuse(),
                LnNext lnext = LnNext()) {
  const float* Wt = W(c, name + ".weight");
  const float* b = W(c, name + ".bias");
  if (c.cfg.linear_layout == 0) {
    GemmArgs a = lin(A, lda, Wt, b, C, ldc, M, N, K, flags);
    a.ln_stats = lnf.stats;
    a.ln_g = lnf.g;
    a.ln_b = lnf.b;
    if (lnext.y) with_lnout(a, c, lnext);
    if (rope_cols) with_rope(a, c, rope_cols);
    if (flags & EPI_RES1) {
      a.R1 = C;
      a.ldr1 = ldc;
    }
    return run1(c, a, aload, s);
  }
  GS_REQUIRE(aload == A_PLAIN, "linear: the literal layout takes fp32 activations");
  GS_REQUIRE(!lnext.y, "linear: the literal layout has no fused LayerNorm output");
  const int Ng = N / groups;
  for (int g = 0; g < groups; ++g) {
    GemmArgs a = lin(A, lda, Wt + (int64_t)g * Ng * K, b ? b + (int64_t)g * Ng : nullptr,
                     C + (int64_t)g * Ng, ldc, M, Ng, K, flags);
    a.ldb = Ng;  // literal: the [Ng, K] buffer read as [K, Ng]
    const int rc_cols = rope_cols - g * Ng;
    if (rc_cols > 0) with_rope(a, c, rc_cols > Ng ? Ng : rc_cols);
    if (flags & EPI_RES1) {
      a.R1 = C + (int64_t)g * Ng;
      a.ldr1 = ldc;
    }
    GemmBatch bt;
    bt.g[0] = a;
    bt.ngroups = 1;
    RC(launch_gemm(bt, A_PLAIN, B_NN, false, s));
  }
  return 0;
}

int layernorm1(const float* x, const float* g, const float* b, float* y, int64_t rows, int D,
               float eps, hipStream_t s, bool y_bf16 = false, float* stats = nullptr) {
  LnBatch bt;
  bt.g[0] = LnArgs{x, g, b, y, rows, D, eps, y_bf16, stats};
  bt.ngroups = 1;
  return launch_layernorm(bt, s);
}

// Column `off` of rows that start at `base`: fp32 elements, or bf16 elements
// when the producing GEMM wrote bf16 (EPI_BF16OUT); row starts and strides
// count elements of the same type.
const float* col_at(const float* base, int64_t off, bool bf16) {
  return bf16 ? (const float*)((const __bf16*)base + off) : base + off;
}

AttnArgs attn_args(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                   int64_t ldv, float* o, int64_t ldo, int B, int H, int N) {
  AttnArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.q_sb = (int64_t)N * ldq;
  a.q_sh = 64;
  a.q_sn = ldq;
  a.k_sb = (int64_t)N * ldk;
  a.k_sh = 64;
  a.k_sn = ldk;
  a.v_sb = (int64_t)N * ldv;
  a.v_sh = 64;
  a.v_sn = ldv;
  a.o_sb = (int64_t)N * ldo;
  a.o_sh = 64;
  a.o_sn = ldo;
  a.B = B;
  a.H = H;
  a.Nq = N;
  a.Nkv = N;
  a.scale = 1.0f / sqrtf(64.0f);
  return a;
}

// MASt3REncoderBlockV2#forward, in place on x [M, De] (M = images * N).
// pre_normed: c.h already holds norm1(x) (the previous block's fc2 wrote it);
// next: the LayerNorm after this block (the next block's norm1 or enc_norm),
// run on the fc2 output rows by the fc2 launch (fp32 products only).
int encoder_block(Ctx& c, int l, float* x, int64_t M, hipStream_t s, bool pre_normed = false,
                  LnNext next = LnNext()) {
  const gs_mastr_config& f = c.cfg;
  const int D = f.enc_dim, H = f.enc_heads;
  const std::string p = "enc_blocks." + std::to_string(l);
  const int rope = f.rope_mode == 1 ? 2 * D : 0;
  // bf16 mode: the LN, attention and fc1 outputs that only feed bf16 GEMMs
  // are stored as bf16 (the same rounding the GEMM's A load applies to fp32)
  const bool hb = f.precision == 1;
  const int aH = hb ? A_PLAIN_H : A_PLAIN;
  // bf16x6 products (precision 2): the norm1 / norm2 apply steps run in the
  // qkv / fc1 A loads, after a statistics-only LayerNorm pass. fp32 products
  // (precision 0) write the normalised rows once and read them as plain
  // rows: large launches then run the 256 x 128 kernel (measured at config 3:
  // encoder fc1 125 -> 136 TFLOP/s, qkv 122 -> 134, with the LayerNorm pass
  // 25 us longer), small ones the direct-to-LDS kernel (one image: qkv 68.8
  // -> 59.1 us, fc1 70.4 -> 67.9 us, the LayerNorm pass ~2 us longer)
  const bool fuse = f.precision == 2 && f.linear_layout == 0;
  const bool fuse_mlp = fuse;
  // fp32 products: the GEMM before each LayerNorm also writes it (EPI_LNOUT,
  // in the split-K reduce pass where the launch splits: one launch and one
  // read of the rows fewer per LayerNorm)
  const bool chain = f.precision == 0 && f.linear_layout == 0;
  GS_REQUIRE(!pre_normed || chain, "encoder block: pre-normalised rows need fp32 products");
  const LnFuse ln1{c.lnst, W(c, p + ".norm1.weight"), W(c, p + ".norm1.bias")};
  const LnFuse ln2{c.lnst, W(c, p + ".norm2.weight"), W(c, p + ".norm2.bias")};
  if (fuse) {
    RC(layernorm1(x, ln1.g, ln1.b, nullptr, M, D, f.ln_eps, s, false, c.lnst));
    RC(linear_mode(c, p + ".attn.qkv", x, D, c.qkv, 3 * D, M, 3 * D, D, 0, s, 3, rope, A_LN,
                   ln1));
  } else {
    if (!pre_normed) RC(layernorm1(x, ln1.g, ln1.b, c.h, M, D, f.ln_eps, s, hb));
    RC(linear_mode(c, p + ".attn.qkv", c.h, D, c.qkv, 3 * D, M, 3 * D, D,
                   hb ? EPI_BF16OUT : 0, s, 3, rope, aH));
  }
  AttnBatch ab;
  ab.g[0] = attn_args(c.qkv, 3 * D, col_at(c.qkv, D, hb), 3 * D, col_at(c.qkv, 2 * D, hb), 3 * D, c.att, D,
                      (int)(M / c.N), H, c.N);
  ab.g[0].o_bf16 = hb;
  ab.g[0].in_bf16 = hb;
  ab.ngroups = 1;
  RC(attention(c, ab, s));
  RC(linear_mode(c, p + ".attn.proj", c.att, D, x, D, M, D, D, EPI_RES1, s, 1, 0, aH, LnFuse(),
                 chain ? LnNext{ln2.g, ln2.b, c.h} : LnNext()));
  if (fuse_mlp) {
    RC(layernorm1(x, ln2.g, ln2.b, nullptr, M, D, f.ln_eps, s, false, c.lnst));
    RC(linear_mode(c, p + ".mlp.fc1", x, D, c.mlp, f.enc_mlp, M, f.enc_mlp, D, EPI_GELU, s, 1, 0,
                   A_LN, ln2));
  } else {
    if (!chain) RC(layernorm1(x, ln2.g, ln2.b, c.h, M, D, f.ln_eps, s, hb));
    RC(linear_mode(c, p + ".mlp.fc1", c.h, D, c.mlp, f.enc_mlp, M, f.enc_mlp, D,
                   EPI_GELU | (hb ? EPI_BF16OUT : 0), s, 1, 0, aH));
  }
  GS_REQUIRE(!next.y || chain, "encoder block: a fused next LayerNorm needs fp32 products");
  RC(linear_mode(c, p + ".mlp.fc2", c.mlp, f.enc_mlp, x, D, M, D, f.enc_mlp, EPI_RES1, s, 1, 0,
                 aH, LnFuse(), next));
  return 0;
}

// MASt3REncoderV2#forward over `nimg` images already unfolded in c.P.
int encoder_from_patches(Ctx& c, int64_t nimg, float* out, hipStream_t s) {
  const gs_mastr_config& f = c.cfg;
  const int D = f.enc_dim, K = 3 * f.patch * f.patch;
  const int64_t M = nimg * c.N;
  if (f.rope_mode == 2) {  // token-level RoPE between the patch embedding and block 0
    RC(linear_mode(c, "patch_embed.proj", c.P, K, c.h, D, M, D, K, 0, s));
    RC(launch_rope_ref_token(c.h, c.x, (int)nimg, c.gh, c.gw, D, f.enc_heads, c.ref_cos,
                             c.ref_sin, c.ref_maxpos, s));
  } else {
    RC(linear_mode(c, "patch_embed.proj", c.P, K, c.x, D, M, D, K, 0, s));
  }
  // fp32 products: each block's fc2 also writes the next LayerNorm (the next
  // block's norm1, after the last block enc_norm into out)
  const bool chain = f.precision == 0 && f.linear_layout == 0 && f.enc_depth > 0;
  for (int l = 0; l < f.enc_depth; ++l) {
    LnNext next;
    if (chain) {
      const std::string nn = "enc_blocks." + std::to_string(l + 1) + ".norm1";
      next = l + 1 < f.enc_depth ? LnNext{W(c, nn + ".weight"), W(c, nn + ".bias"), c.h}
                                 : LnNext{W(c, "enc_norm.weight"), W(c, "enc_norm.bias"), out};
    }
    RC(encoder_block(c, l, c.x, M, s, chain && l > 0, next));
  }
  if (!chain)
    RC(layernorm1(c.x, W(c, "enc_norm.weight"), W(c, "enc_norm.bias"), out, M, D, f.ln_eps, s));
  return 0;
}

// Decoder over both chains. enc [2*B*N, De] (view 1 rows first).
int decoder(Ctx& c, int B, hipStream_t s) {
  const gs_mastr_config& f = c.cfg;
  const int D = f.dec_dim, H = f.dec_heads, De = f.enc_dim;
  const int64_t Mv = (int64_t)B * c.N, M = 2 * Mv;
  const float eps = f.ln_eps;
  const bool rope = f.rope_mode == 1;
  const bool own_memory = f.composite == 1;
  // bf16 mode: LN, attention and fc1 outputs stored as bf16 (see encoder_block)
  const bool hb = f.precision == 1;
  const int aH = hb ? A_PLAIN_H : A_PLAIN;
  {
    GemmArgs a = lin(c.enc, De, W(c, "decoder_embed.weight"), W(c, "decoder_embed.bias"), c.d, D, M,
                     D, De, own_memory ? EPI_DUAL : 0);
    a.C2 = own_memory ? c.dmem : nullptr;
    RC(run1(c, a, A_PLAIN, s));
  }
  for (int l = 0; l < f.dec_depth; ++l) {
    std::string p[2] = {"dec_blocks." + std::to_string(l), "dec_blocks2." + std::to_string(l)};
    float* dc[2] = {c.d, c.d + Mv * D};
    float* hc[2] = {c.h, c.h + Mv * D};
    float* yc[2] = {c.ym, c.ym + Mv * D};
    float* kvc[2] = {c.kv, c.kv + Mv * 2 * D};
    float* qkvc[2] = {c.qkv, c.qkv + Mv * 3 * D};
    float* qc[2] = {c.q, c.q + Mv * D};
    float* ac[2] = {c.att, c.att + Mv * D};
    float* mc[2] = {c.mlp, c.mlp + Mv * f.dec_mlp};
    // LayerNorm of src per chain. bf16x6 products (precision 2): a
    // statistics-only pass, the apply step runs in the next GEMM's A load
    // (A_LN) on src; otherwise the normalised rows are written to dst (fp32
    // products read them as plain rows, on the 256 x 128 kernel where the
    // launch is large and the direct-to-LDS kernel where it is small; one
    // pair: decoder fc1 96.8 -> 85.4 us, qkv 71.2 -> 63.6, kv 53.5 -> 48.9).
    // Sets the next GEMM's A sources (asrc) and loader (al).
    const bool fuse = f.precision == 2 && f.linear_layout == 0;
    const float* asrc[2];
    int al = aH;
    const char* lnm = "";
    // fp32 products: the proj GEMM before norm3 / norm2 writes that
    // LayerNorm of its output rows into hc (EPI_LNOUT); ln2 then only sets
    // the next GEMM's sources (written == true)
    const bool chain = f.precision == 0 && f.linear_layout == 0;
    auto ln2 = [&](const char* nm, float* const* src, float* const* dst, bool written = false) {
      if (written) {
        for (int k = 0; k < 2; ++k) asrc[k] = dst[k];
        al = aH;
        lnm = nm;
        return 0;
      }
      LnBatch bt;
      for (int k = 0; k < 2; ++k) {
        bt.g[k] = LnArgs{src[k], W(c, p[k] + nm + ".weight"), W(c, p[k] + nm + ".bias"),
                         fuse ? nullptr : dst[k], Mv, D, eps, hb,
                         fuse ? c.lnst + 2 * Mv * k : nullptr};
        asrc[k] = fuse ? src[k] : dst[k];
      }
      al = fuse ? A_LN : aH;
      lnm = nm;
      bt.ngroups = 2;
      return launch_layernorm(bt, s);
    };
    auto lnset = [&](GemmArgs& a, int k) {
      if (!fuse) return;
      a.ln_stats = c.lnst + 2 * Mv * k;
      a.ln_g = W(c, p[k] + lnm + ".weight");
      a.ln_b = W(c, p[k] + lnm + ".bias");
    };
    // Cross-attention memory: the other view's state before this block, or
    // (composite 1) this view's decoder_embed output.
    float* other[2] = {dc[1], dc[0]};
    if (own_memory) {
      other[0] = c.dmem;
      other[1] = c.dmem + Mv * D;
    }
    RC(ln2(".norm_y", other, yc));
    {
      GemmArgs a[2];
      for (int k = 0; k < 2; ++k) {
        a[k] = lin(asrc[k], D, c.derived[p[k] + ".kv.weight"], c.derived[p[k] + ".kv.bias"],
                   kvc[k], 2 * D, Mv, 2 * D, D, hb ? EPI_BF16OUT : 0);
        lnset(a[k], k);
        if (rope) with_rope(a[k], c, D);
      }
      RC(run2(c, a[0], a[1], al, s));
    }
    // self-attention
    RC(ln2(".norm1", dc, hc));
    {
      GemmArgs a[2];
      for (int k = 0; k < 2; ++k) {
        a[k] = lin(asrc[k], D, W(c, p[k] + ".attn.qkv.weight"), W(c, p[k] + ".attn.qkv.bias"),
                   qkvc[k], 3 * D, Mv, 3 * D, D, hb ? EPI_BF16OUT : 0);
        lnset(a[k], k);
        if (rope) with_rope(a[k], c, 2 * D);
      }
      RC(run2(c, a[0], a[1], al, s));
      AttnBatch ab;
      for (int k = 0; k < 2; ++k) {
        ab.g[k] = attn_args(qkvc[k], 3 * D, col_at(qkvc[k], D, hb), 3 * D,
                            col_at(qkvc[k], 2 * D, hb), 3 * D, ac[k], D, B, H, c.N);
        ab.g[k].o_bf16 = hb;
        ab.g[k].in_bf16 = hb;
      }
      ab.ngroups = 2;
      RC(attention(c, ab, s));
      for (int k = 0; k < 2; ++k) {
        a[k] = lin(ac[k], D, W(c, p[k] + ".attn.proj.weight"), W(c, p[k] + ".attn.proj.bias"),
                   dc[k], D, Mv, D, D, EPI_RES1);
        a[k].R1 = dc[k];
        a[k].ldr1 = D;
        if (chain)
          with_lnout(a[k], c, LnNext{W(c, p[k] + ".norm3.weight"), W(c, p[k] + ".norm3.bias"), hc[k]});
      }
      RC(run2(c, a[0], a[1], aH, s));
    }
    // cross-attention (query norm3, reference role naming)
    RC(ln2(".norm3", dc, hc, chain));
    {
      GemmArgs a[2];
      for (int k = 0; k < 2; ++k) {
        a[k] = lin(asrc[k], D, W(c, p[k] + ".cross_attn.projq.weight"),
                   W(c, p[k] + ".cross_attn.projq.bias"), qc[k], D, Mv, D, D,
                   hb ? EPI_BF16OUT : 0);
        lnset(a[k], k);
        if (rope) with_rope(a[k], c, D);
      }
      RC(run2(c, a[0], a[1], al, s));
      AttnBatch ab;
      for (int k = 0; k < 2; ++k) {
        ab.g[k] = attn_args(qc[k], D, kvc[k], 2 * D, col_at(kvc[k], D, hb), 2 * D, ac[k], D, B, H,
                            c.N);
        ab.g[k].o_bf16 = hb;
        ab.g[k].in_bf16 = hb;
      }
      ab.ngroups = 2;
      RC(attention(c, ab, s));
      for (int k = 0; k < 2; ++k) {
        a[k] = lin(ac[k], D, W(c, p[k] + ".cross_attn.proj.weight"),
                   W(c, p[k] + ".cross_attn.proj.bias"), dc[k], D, Mv, D, D, EPI_RES1);
        a[k].R1 = dc[k];
        a[k].ldr1 = D;
        if (chain)
          with_lnout(a[k], c, LnNext{W(c, p[k] + ".norm2.weight"), W(c, p[k] + ".norm2.bias"), hc[k]});
      }
      RC(run2(c, a[0], a[1], aH, s));
    }
    // MLP (norm2, reference role naming)
    RC(ln2(".norm2", dc, hc, chain));
    {
      GemmArgs a[2];
      for (int k = 0; k < 2; ++k) {
        a[k] = lin(asrc[k], D, W(c, p[k] + ".mlp.fc1.weight"), W(c, p[k] + ".mlp.fc1.bias"),
                   mc[k], f.dec_mlp, Mv, f.dec_mlp, D, EPI_GELU | (hb ? EPI_BF16OUT : 0));
        lnset(a[k], k);
      }
      RC(run2(c, a[0], a[1], al, s));
      // the DPT hooks snapshot the state after blocks hooks[1] and hooks[2]:
      // the fc2 epilogue stores that block's output a second time
      float* hook = f.dpt_hooks[1] == l + 1 ? c.hook1 : (f.dpt_hooks[2] == l + 1 ? c.hook2 : nullptr);
      float* hook2 = (f.dpt_hooks[1] == l + 1 && f.dpt_hooks[2] == l + 1) ? c.hook2 : nullptr;
      for (int k = 0; k < 2; ++k) {
        a[k] = lin(mc[k], f.dec_mlp, W(c, p[k] + ".mlp.fc2.weight"), W(c, p[k] + ".mlp.fc2.bias"),
                   dc[k], D, Mv, D, f.dec_mlp, EPI_RES1 | (hook ? EPI_DUAL : 0));
        a[k].R1 = dc[k];
        a[k].ldr1 = D;
        if (hook) a[k].C2 = hook + (int64_t)k * Mv * D;
      }
      RC(run2(c, a[0], a[1], aH, s));
      if (hook2)  // both hooks on the same block
        GS_CHECK_HIP(hipMemcpyAsync(hook2, hook, M * D * sizeof(float), hipMemcpyDeviceToDevice, s));
    }
  }
  RC(layernorm1(c.d, W(c, "dec_norm.weight"), W(c, "dec_norm.bias"), c.dfin, M, D, eps, s));
  return 0;
}

// The two views' DPT heads (and descriptor heads) have identical shapes and
// separate weights, so each of their convolutions runs as ONE grouped launch
// (z = head): the 1/32- and 1/16-scale convolutions alone would fill a
// fraction of the GPU.
struct Heads {
  int n = 0;       // 1 or 2 heads in this launch sequence
  int id[2];       // checkpoint head number (1 or 2) of group slot v
  std::string pre(int v) const { return "downstream_head" + std::to_string(id[v]); }
};

// Conv as implicit GEMM on NHWC tensors [imgs, H, W, Cin], one problem per
// head; `suffix` is the weight name after the head prefix (weights of 3x3
// convs are already OHWI).
int conv(Ctx& c, const Heads& hs, const std::string& suffix, const float* const x[2], int imgs,
         int H, int W_, int Cin, int Cout, int k, int stride, int pad, bool bias,
         float* const y[2], int flags, bool relu_in, hipStream_t s,
         const float* const r1[2] = nullptr, const float* const r2[2] = nullptr,
         bool in_bf16 = false, float* const yh[2] = nullptr) {
  const int Ho = (H + 2 * pad - k) / stride + 1, Wo = (W_ + 2 * pad - k) / stride + 1;
  GemmBatch b;
  b.ngroups = hs.n;
  for (int v = 0; v < hs.n; ++v) {
    const std::string name = hs.pre(v) + suffix;
    GemmArgs a = lin(x[v], Cin, W(c, name + ".weight"), bias ? W(c, name + ".bias") : nullptr,
                     y[v], Cout, (int64_t)imgs * Ho * Wo, Cout, k * k * Cin, flags);
    a.cH = H;
    a.cW = W_;
    a.cCin = Cin;
    a.ck = k;
    a.ckw = k;
    a.cs = stride;
    a.cp = pad;
    a.cHo = Ho;
    a.cWo = Wo;
    if (r1) {
      a.flags |= EPI_RES1;
      a.R1 = r1[v];
      a.ldr1 = Cout;
    }
    if (r2) {
      a.flags |= EPI_RES2;
      a.R2 = r2[v];
      a.ldr2 = Cout;
    }
    if (yh) {  // also bf16(max(y, 0)) for an RCU conv1 that reads it
      a.flags |= EPI_DUAL | EPI_DUAL_RELU_H;
      a.C2 = yh[v];
    }
    b.g[v] = a;
  }
  const bool pointwise = (k == 1 && stride == 1 && pad == 0);
  // in_bf16: x holds bf16 (its producer wrote it so in the bf16 mode)
  GS_REQUIRE(!in_bf16 || (!relu_in && c.cfg.precision == 1),
             "conv: a bf16 input needs a conv without ReLU prologue in the bf16 mode");
  const int al = pointwise ? (in_bf16 ? A_PLAIN_H : A_PLAIN) : (in_bf16 ? A_CONV_H : A_CONV);
  return gemm(c, b, al, relu_in, s);
}

// ConvTranspose (k == s) from [rows, Cin] token tensors on the gh x gw grid;
// bf16 mode: in_bf16 / out_bf16 read / write bf16 rows.
int convt(Ctx& c, const Heads& hs, const std::string& suffix, const float* const x[2], int imgs,
          int Cin, int Cout, int k, float* const y[2], hipStream_t s, bool in_bf16 = false,
          bool out_bf16 = false) {
  GS_REQUIRE(!(in_bf16 || out_bf16) || c.cfg.precision == 1,
             "convt: bf16 rows are the bf16 mode's");
  GemmBatch b;
  b.ngroups = hs.n;
  for (int v = 0; v < hs.n; ++v) {
    const std::string name = hs.pre(v) + suffix;
    GemmArgs a = lin(x[v], Cin, c.derived[name + ".weight"], c.derived[name + ".bias"], y[v], 0,
                     (int64_t)imgs * c.N, k * k * Cout, Cin,
                     EPI_SCATTER | (out_bf16 ? EPI_BF16OUT : 0));
    a.sc_r = k;
    a.sc_C = Cout;
    a.sc_Cout = Cout;
    a.sc_gh = c.gh;
    a.sc_gw = c.gw;
    b.g[v] = a;
  }
  return gemm(c, b, in_bf16 ? A_PLAIN_H : A_PLAIN, false, s);
}

// FeatureFusionBlock: out = out_conv(up2(RCU2(x0 (+ RCU1(x1))))). The 1x1
// out_conv and the bilinear x2 upsample commute (both are linear and the
// bilinear weights of each output pixel sum to one, so the bias passes
// through), so out_conv runs at the input resolution: a quarter of its FLOPs
// and of the upsample's input traffic. Differences are fp32 rounding only.
// bf16 mode: each RCU's conv1 output feeds only its conv2, so it is written in
// bf16 (the rounding conv2's A load would apply) and conv2 reads it so; with
// out_bf16 the final upsample does the same for a single bf16 consumer. Each
// RCU conv1 reads bf16(max(x, 0)) of its input, written beside x by x's
// producer (x0h / x1h for x0 / x1; RCU1's conv2 writes that of the sum into
// c.t, free until RCU2's conv2 overwrites it).
int fusion(Ctx& c, const Heads& hs, const std::string& suffix, const float* const x0[2],
           const float* const x1[2], int B, int H, int W_, float* const out[2], hipStream_t s,
           bool out_bf16 = false, const float* const x0h[2] = nullptr,
           const float* const x1h[2] = nullptr) {
  const int F = c.cfg.dpt_feat;
  const bool hb = c.cfg.precision == 1;
  const int ub = hb ? EPI_BF16OUT : 0;
  const float* sum[2] = {x0[0], x0[1]};
  const float* sumh[2] = {x0h ? x0h[0] : nullptr, x0h ? x0h[1] : nullptr};
  if (x1) {
    GS_REQUIRE(!hb || x1h, "fusion: the bf16 mode needs the ReLU'd bf16 copy of x1");
    if (hb)
      RC(conv(c, hs, suffix + ".resConfUnit1.conv1", x1h, B, H, W_, F, F, 3, 1, 1, true, c.u,
              EPI_RELU | ub, false, s, nullptr, nullptr, true));
    else
      RC(conv(c, hs, suffix + ".resConfUnit1.conv1", x1, B, H, W_, F, F, 3, 1, 1, true, c.u,
              EPI_RELU, true, s));
    const float* uin[2] = {c.u[0], c.u[1]};
    RC(conv(c, hs, suffix + ".resConfUnit1.conv2", uin, B, H, W_, F, F, 3, 1, 1, true, c.s, 0,
            false, s, x1, x0, hb, hb ? c.t : nullptr));
    sum[0] = c.s[0];
    sum[1] = c.s[1];
    sumh[0] = c.t[0];
    sumh[1] = c.t[1];
  }
  if (hb) {
    GS_REQUIRE(sumh[0] && sumh[1], "fusion: the bf16 mode needs the ReLU'd bf16 copy of x0");
    RC(conv(c, hs, suffix + ".resConfUnit2.conv1", sumh, B, H, W_, F, F, 3, 1, 1, true, c.u,
            EPI_RELU | ub, false, s, nullptr, nullptr, true));
  } else {
    RC(conv(c, hs, suffix + ".resConfUnit2.conv1", sum, B, H, W_, F, F, 3, 1, 1, true, c.u,
            EPI_RELU, true, s));
  }
  const float* uin[2] = {c.u[0], c.u[1]};
  // RCU2's output feeds only the 1x1 out_conv: bf16 in the bf16 mode
  RC(conv(c, hs, suffix + ".resConfUnit2.conv2", uin, B, H, W_, F, F, 3, 1, 1, true, c.t, ub, false,
          s, sum, nullptr, hb));
  const float* tin[2] = {c.t[0], c.t[1]};
  // a bf16 output (single bf16 consumer): out_conv's rows, which feed only
  // the upsample, are bf16 too
  const bool ob = out_bf16 && hb;
  RC(conv(c, hs, suffix + ".out_conv", tin, B, H, W_, F, F, 1, 1, 0, true, c.up,
          ob ? EPI_BF16OUT : 0, false, s, nullptr, nullptr, hb));
  for (int v = 0; v < hs.n; ++v)
    RC(launch_upsample2x(c.up[v], B, H, W_, F, out[v], s, ob, ob));
  return 0;
}

// DPT heads; hooks are per group slot row blocks of [B*N, dim] tensors.
int dpt_heads(Ctx& c, const Heads& hs, const float* const e[2], const float* const h6[2],
              const float* const h9[2], const float* const dfin[2], int B, float* const pts[2],
              float* const conf[2], hipStream_t s) {
  const gs_mastr_config& f = c.cfg;
  const int F = f.dpt_feat, gh = c.gh, gw = c.gw;
  const std::string ap = ".dpt.act_postprocess.";
  const int* d = f.dpt_dims;
  const float* t0c[2] = {c.t0[0], c.t0[1]};
  float* act[4][2];
  for (int i = 0; i < 4; ++i)
    for (int v = 0; v < 2; ++v) act[i][v] = c.act[v][i];
  // act_postprocess. bf16 mode: every output here feeds a single bf16 GEMM
  // (the next act_postprocess step or a layer_rn conv), so it is written in
  // bf16 and read so
  const bool hb = f.precision == 1;
  const int ub = hb ? EPI_BF16OUT : 0;
  RC(conv(c, hs, ap + "0.0", e, B, gh, gw, f.enc_dim, d[0], 1, 1, 0, true, c.t0, ub, false, s));
  RC(convt(c, hs, ap + "0.1", t0c, B, d[0], d[0], 4, act[0], s, hb, hb));
  RC(conv(c, hs, ap + "1.0", h6, B, gh, gw, f.dec_dim, d[1], 1, 1, 0, true, c.t0, ub, false, s));
  RC(convt(c, hs, ap + "1.1", t0c, B, d[1], d[1], 2, act[1], s, hb, hb));
  RC(conv(c, hs, ap + "2.0", h9, B, gh, gw, f.dec_dim, d[2], 1, 1, 0, true, act[2], ub, false, s));
  RC(conv(c, hs, ap + "3.0", dfin, B, gh, gw, f.dec_dim, d[3], 1, 1, 0, true, c.t0, ub, false, s));
  RC(conv(c, hs, ap + "3.1", t0c, B, gh, gw, d[3], d[3], 3, 2, 1, true, act[3], ub, false, s,
          nullptr, nullptr, hb));
  const int ah[4] = {4 * gh, 2 * gh, gh, gh / 2}, aw[4] = {4 * gw, 2 * gw, gw, gw / 2};
  float* L[4][2];
  for (int i = 0; i < 4; ++i) {
    for (int v = 0; v < 2; ++v) L[i][v] = c.L[v][i];
    const float* ain[2] = {act[i][0], act[i][1]};
    float* Lh[2] = {c.Lh[0][i], c.Lh[1][i]};
    RC(conv(c, hs, ".dpt.scratch.layer" + std::to_string(i + 1) + "_rn", ain, B, ah[i], aw[i], d[i],
            F, 3, 1, 1, false, L[i], 0, false, s, nullptr, nullptr, hb, hb ? Lh : nullptr));
  }
  const float* Lhc[4][2];
  for (int i = 0; i < 4; ++i)
    for (int v = 0; v < 2; ++v) Lhc[i][v] = c.Lh[v][i];
  const std::string rp = ".dpt.scratch.refinenet";
  const float* Lc[4][2];
  for (int i = 0; i < 4; ++i)
    for (int v = 0; v < 2; ++v) Lc[i][v] = L[i][v];
  const float* rAc[2] = {c.rA[0], c.rA[1]};
  const float* rBc[2] = {c.rB[0], c.rB[1]};
  RC(fusion(c, hs, rp + "4", Lc[3], nullptr, B, ah[3], aw[3], c.rA, s, false, Lhc[3]));
  RC(fusion(c, hs, rp + "3", rAc, Lc[2], B, ah[2], aw[2], c.rB, s, false, nullptr, Lhc[2]));
  RC(fusion(c, hs, rp + "2", rBc, Lc[1], B, ah[1], aw[1], c.rA, s, false, nullptr, Lhc[1]));
  // refinenet1's output feeds only head.0: bf16 in the bf16 mode
  RC(fusion(c, hs, rp + "1", rAc, Lc[0], B, ah[0], aw[0], c.rB, s, true, nullptr, Lhc[0]));
  const int h1 = 2 * ah[0], w1 = 2 * aw[0];
  // bf16 mode: head.0's output feeds only the upsample, and the
  // full-resolution upsample feeds only the next conv, so both are written in
  // bf16 (the rounding that conv's A load would apply) and read so
  RC(conv(c, hs, ".dpt.head.0", rBc, B, h1, w1, F, F / 2, 3, 1, 1, true, c.hd0,
          hb ? EPI_BF16OUT : 0, false, s, nullptr, nullptr, hb));
  for (int v = 0; v < hs.n; ++v)
    RC(launch_upsample2x(c.hd0[v], B, h1, w1, F / 2, c.hup[v], s, hb, hb));
  const float* hupc[2] = {c.hup[0], c.hup[1]};
  // head.2's ReLU output feeds only head.4 (head_out): bf16 in the bf16 mode
  RC(conv(c, hs, ".dpt.head.2", hupc, B, 2 * h1, 2 * w1, F / 2, f.head_mid, 3, 1, 1, true, c.hd2,
          EPI_RELU | (hb ? EPI_BF16OUT : 0), false, s, nullptr, nullptr, hb));
  for (int v = 0; v < hs.n; ++v)
    RC(launch_head_out(c.hd2[v], (int64_t)B * 4 * h1 * w1, f.head_mid,
                       W(c, hs.pre(v) + ".dpt.head.4.weight"), W(c, hs.pre(v) + ".dpt.head.4.bias"),
                       pts[v], conf[v], false, s, hb));
  return 0;
}

// The reference's stub DPTHead#forward (src/mastr/decoder_v2.cr:502-530) on
// the patch grid: layer4_rn (3x3, no bias) -> refinenet4 without skip (two
// conv-ReLU-conv+x units, src/mastr/decoder_v2.cr:365-370, then the 1x1
// out_conv) -> ReLU -> head.0 -> ReLU -> head.2 -> head.4 -> pts, sigmoid conf.
// The ReLUs before head.0 / head.2 run as the convolutions' input prologue.
int dpt_ref_heads(Ctx& c, const Heads& hs, const float* const dfin[2], int B,
                  float* const pts[2], float* const conf[2], hipStream_t s) {
  const gs_mastr_config& f = c.cfg;
  const int F = f.dpt_feat, gh = c.gh, gw = c.gw;
  float* L[2] = {c.L[0][2], c.L[1][2]};
  RC(conv(c, hs, ".dpt.scratch.layer4_rn", dfin, B, gh, gw, f.dec_dim, F, 3, 1, 1, false, L, 0,
          false, s));
  const std::string rp = ".dpt.scratch.refinenet4";
  const float* Lc[2] = {L[0], L[1]};
  const float* uc[2] = {c.u[0], c.u[1]};
  RC(conv(c, hs, rp + ".resConfUnit1.conv1", Lc, B, gh, gw, F, F, 3, 1, 1, true, c.u, EPI_RELU,
          false, s));
  RC(conv(c, hs, rp + ".resConfUnit1.conv2", uc, B, gh, gw, F, F, 3, 1, 1, true, c.s, 0, false, s,
          Lc));
  const float* sc[2] = {c.s[0], c.s[1]};
  RC(conv(c, hs, rp + ".resConfUnit2.conv1", sc, B, gh, gw, F, F, 3, 1, 1, true, c.u, EPI_RELU,
          false, s));
  RC(conv(c, hs, rp + ".resConfUnit2.conv2", uc, B, gh, gw, F, F, 3, 1, 1, true, c.t, 0, false, s,
          sc));
  const float* tc[2] = {c.t[0], c.t[1]};
  RC(conv(c, hs, rp + ".out_conv", tc, B, gh, gw, F, F, 1, 1, 0, true, c.up, 0, false, s));
  const float* upc[2] = {c.up[0], c.up[1]};
  RC(conv(c, hs, ".dpt.head.0", upc, B, gh, gw, F, F / 2, 3, 1, 1, true, c.hd0, 0, true, s));
  const float* h0c[2] = {c.hd0[0], c.hd0[1]};
  RC(conv(c, hs, ".dpt.head.2", h0c, B, gh, gw, F / 2, f.head_mid, 3, 1, 1, true, c.hd2, 0, true,
          s));
  for (int v = 0; v < hs.n; ++v)
    RC(launch_head_out(c.hd2[v], (int64_t)B * c.N, f.head_mid,
                       W(c, hs.pre(v) + ".dpt.head.4.weight"), W(c, hs.pre(v) + ".dpt.head.4.bias"),
                       pts[v], conf[v], true, s));
  return 0;
}

// Local-feature descriptors: MLP(concat(enc, dec)) + pixel shuffle, per head.
int local_features(Ctx& c, const Heads& hs, const float* const e[2], const float* const dfin[2],
                   int B, float* const desc[2], hipStream_t s) {
  const gs_mastr_config& f = c.cfg;
  const int Din = f.enc_dim + f.dec_dim;
  const int64_t Mv = (int64_t)B * c.N;
  const int r = f.patch;
  GemmBatch b1, b2;
  b1.ngroups = b2.ngroups = hs.n;
  for (int v = 0; v < hs.n; ++v) {
    const std::string p = hs.pre(v) + ".head_local_features";
    // bf16 mode: the hidden activations feed only fc2, so fc1 writes them in
    // bf16 and fc2 reads them so (the 256 x 128 bf16 kernel, scatter epilogue)
    GemmArgs a = lin(e[v], f.enc_dim, W(c, p + ".fc1.weight"), W(c, p + ".fc1.bias"), c.lf[v],
                     f.lf_hidden, Mv, f.lf_hidden, Din,
                     EPI_GELU | (f.precision == 1 ? EPI_BF16OUT : 0));
    a.A2 = dfin[v];
    a.lda2 = f.dec_dim;
    a.K1 = f.enc_dim;
    b1.g[v] = a;
    GemmArgs g = lin(c.lf[v], f.lf_hidden, c.derived[p + ".fc2.weight"],
                     c.derived[p + ".fc2.bias"], desc[v], 0, Mv, r * r * f.desc_dim, f.lf_hidden,
                     EPI_SCATTER);
    g.sc_r = r;
    g.sc_C = f.desc_dim;
    g.sc_Cout = f.desc_dim;
    g.sc_gh = c.gh;
    g.sc_gw = c.gw;
    b2.g[v] = g;
  }
  RC(gemm(c, b1, A_CONCAT, false, s));
  return gemm(c, b2, f.precision == 1 ? A_PLAIN_H : A_PLAIN, false, s);
}

// ---------------------------------------------------------------------------
// Weight placement
// ---------------------------------------------------------------------------
int place_weight(Ctx& c, const std::string& name, const float* host, int64_t n) {
  auto it = c.w.find(name);
  GS_REQUIRE(it != c.w.end(), "set_weight: unknown weight " + name);
  DevW& dw = it->second;
  GS_REQUIRE(n == dw.host_numel, "set_weight: numel mismatch for " + name);
  std::vector<float> tmp;
  const float* src = host;
  int64_t count = n;
  float* dst = dw.ptr;
  switch (dw.place) {
    case P_PLAIN:
      break;
    case P_CONV: {  // a = Cout, b = Cin, c = k
      const int64_t Co = dw.a, Ci = dw.b, k = dw.c;
      tmp.resize(n);
      for (int64_t oc = 0; oc < Co; ++oc)
        for (int64_t ic = 0; ic < Ci; ++ic)
          for (int64_t kh = 0; kh < k; ++kh)
            for (int64_t kw = 0; kw < k; ++kw)
              tmp[((oc * k + kh) * k + kw) * Ci + ic] = host[((oc * Ci + ic) * k + kh) * k + kw];
      src = tmp.data();
      break;
    }
    case P_CONVT_W: {  // a = Cin, b = Cout, c = k
      const int64_t Ci = dw.a, Co = dw.b, k = dw.c;
      tmp.resize(n);
      for (int64_t ic = 0; ic < Ci; ++ic)
        for (int64_t oc = 0; oc < Co; ++oc)
          for (int64_t i = 0; i < k; ++i)
            for (int64_t j = 0; j < k; ++j)
              tmp[((i * k + j) * Co + oc) * Ci + ic] = host[((ic * Co + oc) * k + i) * k + j];
      src = tmp.data();
      break;
    }
    case P_CONVT_B: {  // a = Cout, c = k
      const int64_t Co = dw.a, k = dw.c;
      tmp.resize(k * k * Co);
      for (int64_t s = 0; s < k * k; ++s)
        for (int64_t oc = 0; oc < Co; ++oc) tmp[s * Co + oc] = host[oc];
      src = tmp.data();
      count = (int64_t)tmp.size();
      break;
    }
    case P_KV:  // a = element offset within the concatenated buffer
      dst = dw.ptr + dw.a;
      break;
    case P_DESC_W:    // a = r (patch), b = desc channels, c = K
    case P_DESC_B: {  // rows c*r*r + s (s = i*r + j) -> s*desc + c, c < desc
      const int64_t r2 = dw.a * dw.a, C = dw.b, K = dw.place == P_DESC_W ? dw.c : 1;
      tmp.resize(r2 * C * K);
      for (int64_t s = 0; s < r2; ++s)
        for (int64_t ch = 0; ch < C; ++ch)
          memcpy(&tmp[(s * C + ch) * K], host + (ch * r2 + s) * K, K * sizeof(float));
      src = tmp.data();
      count = (int64_t)tmp.size();
      break;
    }
  }
  GS_CHECK_HIP(hipMemcpy(dst, src, count * sizeof(float), hipMemcpyHostToDevice));
  c.bf16_dirty = true;
  return 0;
}

// Refresh the bf16 weight mirror (precision 1) or split planes (precision 2)
// after weight updates.
int sync_bf16(Ctx& c, hipStream_t s) {
  if (c.cfg.precision == 0 || !c.bf16_dirty) return 0;
  const int64_t n = (int64_t)(c.warena_size / 4);
  if (c.cfg.precision == 1)
    RC(launch_f32_to_bf16((const float*)c.warena, c.wbf16, n, s));
  else
    RC(launch_f32_to_bf16x3((const float*)c.warena, c.wbf16, n, n, s));
  c.bf16_dirty = false;
  return 0;
}

int build_weights(Ctx& c) {
  const gs_mastr_config& f = c.cfg;
  // sizes: placed tensors + derived buffers
  size_t total = 0;
  std::vector<std::pair<std::string, int64_t>> derived_sizes;
  for (int chain = 0; chain < 2; ++chain)
    for (int l = 0; l < f.dec_depth; ++l) {
      const std::string p = (chain ? "dec_blocks2." : "dec_blocks.") + std::to_string(l);
      derived_sizes.push_back({p + ".kv.weight", (int64_t)2 * f.dec_dim * f.dec_dim});
      derived_sizes.push_back({p + ".kv.bias", (int64_t)2 * f.dec_dim});
    }
  for (int hd = 1; hd <= 2; ++hd) {
    const std::string p = "downstream_head" + std::to_string(hd);
    const int64_t r2 = (int64_t)f.patch * f.patch;
    derived_sizes.push_back({p + ".head_local_features.fc2.weight", r2 * f.desc_dim * f.lf_hidden});
    derived_sizes.push_back({p + ".head_local_features.fc2.bias", r2 * f.desc_dim});
    for (int i = 0; i < 2; ++i) {
      const int64_t d = f.dpt_dims[i], k = i == 0 ? 4 : 2;
      const std::string n = p + ".dpt.act_postprocess." + std::to_string(i) + ".1";
      derived_sizes.push_back({n + ".weight", k * k * d * d});
      derived_sizes.push_back({n + ".bias", k * k * d});
    }
  }
  for (auto& wi : c.inv.w) total += align256(numel(wi) * sizeof(float));
  for (auto& ds : derived_sizes) total += align256(ds.second * sizeof(float));
  GS_CHECK_HIP(hipMalloc(&c.warena, total));
  c.warena_size = total;
  if (f.precision == 1) GS_CHECK_HIP(hipMalloc(&c.wbf16, total / 2));
  if (f.precision == 2) GS_CHECK_HIP(hipMalloc(&c.wbf16, 3 * (total / 2)));
  char* cur = c.warena;
  auto take = [&](int64_t nfl) {
    float* p = (float*)cur;
    cur += align256(nfl * sizeof(float));
    return p;
  };
  for (auto& ds : derived_sizes) c.derived[ds.first] = take(ds.second);
  for (auto& wi : c.inv.w) {
    DevW dw;
    dw.host_numel = numel(wi);
    const std::string& n = wi.name;
    auto ends = [&](const std::string& suf) {
      return n.size() >= suf.size() && n.compare(n.size() - suf.size(), suf.size(), suf) == 0;
    };
    const bool is_kv = n.find(".cross_attn.projk.") != std::string::npos ||
                       n.find(".cross_attn.projv.") != std::string::npos;
    const bool is_desc = n.find(".head_local_features.fc2.") != std::string::npos;
    const bool is_convt = n.find(".act_postprocess.0.1.") != std::string::npos ||
                          n.find(".act_postprocess.1.1.") != std::string::npos;
    if (is_kv) {
      const bool is_v = n.find(".projv.") != std::string::npos;
      const std::string blk = n.substr(0, n.find(".cross_attn."));
      const bool w = ends(".weight");
      dw.ptr = c.derived[blk + (w ? ".kv.weight" : ".kv.bias")];
      dw.place = P_KV;
      dw.a = is_v ? dw.host_numel : 0;
      // also register the plain name so W() finds projk / projv directly
      c.w[n] = dw;
      continue;
    }
    if (is_desc) {
      const bool w = ends(".weight");
      dw.ptr = c.derived[n];
      dw.place = w ? P_DESC_W : P_DESC_B;
      dw.a = f.patch;
      dw.b = f.desc_dim;
      dw.c = f.lf_hidden;
      c.w[n] = dw;
      continue;
    }
    if (is_convt) {
      const bool w = ends(".weight");
      dw.ptr = c.derived[n];
      dw.place = w ? P_CONVT_W : P_CONVT_B;
      dw.a = wi.shape[0];
      dw.b = w ? wi.shape[1] : 0;
      dw.c = n.find(".0.1.") != std::string::npos ? 4 : 2;
      if (!w) dw.a = wi.shape[0];
      c.w[n] = dw;
      continue;
    }
    dw.ptr = take(dw.host_numel);
    if (wi.shape[3] > 1 && n != "patch_embed.proj.weight") {
      dw.place = P_CONV;
      dw.a = wi.shape[0];
      dw.b = wi.shape[1];
      dw.c = wi.shape[2];
    }
    c.w[n] = dw;
  }
  return 0;
}

int build_workspace(Ctx& c) {
  const gs_mastr_config& f = c.cfg;
  const int64_t B = c.max_pairs, N = c.N;
  const int64_t M = 2 * B * N;  // both views' tokens
  const int64_t De = f.enc_dim, Dd = f.dec_dim, F = f.dpt_feat;
  const int64_t dmax = std::max(std::max(f.dpt_dims[0], f.dpt_dims[1]),
                                std::max(f.dpt_dims[2], f.dpt_dims[3]));
  const int64_t Dm = std::max(De, Dd);
  std::vector<std::pair<float**, int64_t>> req = {
      {&c.P, M * 3 * f.patch * f.patch},
      {&c.x, M * De},
      {&c.h, M * Dm},
      {&c.qkv, M * 3 * Dm},
      {&c.att, M * Dm},
      {&c.mlp, M * std::max(f.enc_mlp, f.dec_mlp)},
      {&c.enc, M * De},
      {&c.d, M * Dd},
      {&c.ym, M * Dd},
      {&c.kv, M * 2 * Dd},
      {&c.q, M * Dd},
      {&c.hook1, M * Dd},
      {&c.hook2, M * Dd},
      {&c.dfin, M * Dd},
      {&c.lnst, 2 * M},
      {&c.dmem, f.composite == 1 ? M * Dd : 0},
      {&c.splitk, kSplitkElems},
      {&c.rope_cos, 512 * 16},
      {&c.rope_sin, 512 * 16},
      {&c.ref_cos, 512 * (De / f.enc_heads / 2)},
      {&c.ref_sin, 512 * (De / f.enc_heads / 2)},
  };
  const int64_t hbuf = f.precision == 1 ? 1 : 0;  // bf16-mode-only buffers
  for (int v = 0; v < 2; ++v) {  // DPT / descriptor heads, B images each
    const std::vector<std::pair<float**, int64_t>> head = {
        {&c.t0[v], B * N * dmax},
        {&c.act[v][0], B * 16 * N * f.dpt_dims[0]},
        {&c.act[v][1], B * 4 * N * f.dpt_dims[1]},
        {&c.act[v][2], B * N * f.dpt_dims[2]},
        {&c.act[v][3], B * N / 4 * f.dpt_dims[3]},
        {&c.L[v][0], B * 16 * N * F},
        {&c.L[v][1], B * 4 * N * F},
        {&c.L[v][2], B * N * F},
        {&c.L[v][3], B * N / 4 * F},
        {&c.Lh[v][0], hbuf * B * 8 * N * F},  // bf16: half the floats of L
        {&c.Lh[v][1], hbuf * B * 2 * N * F},
        {&c.Lh[v][2], hbuf * (B * N * F + 1) / 2},
        {&c.Lh[v][3], hbuf * (B * N / 4 * F + 1) / 2},
        {&c.u[v], B * 16 * N * F},
        {&c.s[v], B * 16 * N * F},
        {&c.t[v], B * 16 * N * F},
        {&c.up[v], B * 64 * N * F},
        {&c.rA[v], B * 64 * N * F},
        {&c.rB[v], B * 64 * N * F},
        {&c.hd0[v], B * 64 * N * (F / 2)},
        {&c.hup[v], B * 256 * N * (F / 2)},
        {&c.hd2[v], B * 256 * N * f.head_mid},
        {&c.lf[v], B * N * f.lf_hidden},
    };
    req.insert(req.end(), head.begin(), head.end());
  }
  size_t total = 0;
  for (auto& r : req) total += align256(r.second * sizeof(float));
  GS_CHECK_HIP(hipMalloc(&c.arena, total));
  c.arena_size = total;
  char* cur = c.arena;
  for (auto& r : req) {
    *r.first = (float*)cur;
    cur += align256(r.second * sizeof(float));
  }
  std::vector<float> hc(512 * 16), hs(512 * 16);
  rope_table_host(512, f.rope_base, hc.data(), hs.data());
  GS_CHECK_HIP(hipMemcpy(c.rope_cos, hc.data(), hc.size() * 4, hipMemcpyHostToDevice));
  GS_CHECK_HIP(hipMemcpy(c.rope_sin, hs.data(), hs.size() * 4, hipMemcpyHostToDevice));
  const int hd = f.enc_dim / f.enc_heads;
  c.ref_maxpos = 512;
  std::vector<float> rc(512 * (hd / 2)), rs(512 * (hd / 2));
  rope_ref_table_host(512, hd, f.rope_base, rc.data(), rs.data());
  GS_CHECK_HIP(hipMemcpy(c.ref_cos, rc.data(), rc.size() * 4, hipMemcpyHostToDevice));
  GS_CHECK_HIP(hipMemcpy(c.ref_sin, rs.data(), rs.size() * 4, hipMemcpyHostToDevice));
  return 0;
}

int validate_config(const gs_mastr_config& f) {
  GS_REQUIRE(f.patch > 0 && f.patch % 4 == 0 && f.img_h % f.patch == 0 && f.img_w % f.patch == 0,
             "config: image must be a multiple of the patch size (patch % 4 == 0)");
  const int gh = f.img_h / f.patch, gw = f.img_w / f.patch;
  GS_REQUIRE(gh % 2 == 0 && gw % 2 == 0 && gh <= 512 && gw <= 512, "config: patch grid must be even");
  GS_REQUIRE(f.enc_heads > 0 && f.enc_dim == 64 * f.enc_heads, "config: encoder head dim must be 64");
  GS_REQUIRE(f.dec_heads > 0 && f.dec_dim == 64 * f.dec_heads, "config: decoder head dim must be 64");
  GS_REQUIRE(f.enc_mlp % 32 == 0 && f.dec_mlp % 32 == 0 && f.lf_hidden % 32 == 0,
             "config: hidden sizes must be multiples of 32");
  GS_REQUIRE(f.dpt_feat % 64 == 0 && f.head_mid % 32 == 0, "config: DPT widths must be multiples of 64/32");
  for (int i = 0; i < 4; ++i) GS_REQUIRE(f.dpt_dims[i] % 32 == 0, "config: DPT dims must be multiples of 32");
  GS_REQUIRE(f.dpt_hooks[0] == 0 && f.dpt_hooks[3] == f.dec_depth && f.dpt_hooks[1] >= 1 &&
                 f.dpt_hooks[1] <= f.dec_depth && f.dpt_hooks[2] >= 1 && f.dpt_hooks[2] <= f.dec_depth,
             "config: hooks must be {0, a, b, dec_depth}");
  GS_REQUIRE(f.desc_dim > 0 && (f.patch * f.patch * f.desc_dim) % 32 == 0, "config: bad desc_dim");
  GS_REQUIRE(f.linear_layout == 0 || f.linear_layout == 1, "config: linear_layout must be 0 or 1");
  GS_REQUIRE(f.rope_mode >= 0 && f.rope_mode <= 2, "config: rope_mode must be 0, 1 or 2");
  GS_REQUIRE(f.precision == 0 || ((f.precision == 1 || f.precision == 2) && f.linear_layout == 0),
             "config: precision must be 0 (fp32), 1 (bf16 MFMA) or 2 (fp32 through bf16x6), "
             "1 and 2 with linear_layout 0");
  GS_REQUIRE(f.enc_dim % 32 == 0 && f.dec_dim % 32 == 0, "config: dims must be multiples of 32");
  GS_REQUIRE(f.composite == 0 || f.composite == 1, "config: composite must be 0 or 1");
  GS_REQUIRE(f.composite == 0 || f.dpt_dims[3] == f.dec_dim,
             "config: composite 1 applies layer4_rn to the decoder output (dpt_dims[3] == dec_dim)");
  return 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

void gs_mastr_default_config(gs_mastr_config* c) {
  memset(c, 0, sizeof(*c));
  c->img_h = 384;
  c->img_w = 512;
  c->patch = 16;
  c->enc_dim = 1024;
  c->enc_depth = 24;
  c->enc_heads = 16;
  c->enc_mlp = 4096;
  c->dec_dim = 768;
  c->dec_depth = 12;
  c->dec_heads = 12;
  c->dec_mlp = 3072;
  c->dpt_feat = 256;
  c->dpt_dims[0] = 96;
  c->dpt_dims[1] = 192;
  c->dpt_dims[2] = 384;
  c->dpt_dims[3] = 768;
  c->dpt_hooks[0] = 0;
  c->dpt_hooks[1] = 6;
  c->dpt_hooks[2] = 9;
  c->dpt_hooks[3] = 12;
  c->head_mid = 128;
  c->lf_hidden = 7168;
  c->desc_dim = 24;
  c->ln_eps = 1e-6f;
  c->rope_base = 100.0f;
  c->linear_layout = 0;
  c->rope_mode = 1;
  c->precision = 0;
}

int32_t gs_mastr_weight_count(const gs_mastr_config* cfg) {
  return (int32_t)make_inventory(*cfg).w.size();
}

int32_t gs_mastr_weight_info(const gs_mastr_config* cfg, int32_t i, char* name_out,
                             int32_t name_cap, int64_t shape_out[4], int32_t* kind_out) {
  Inventory inv = make_inventory(*cfg);
  if (i < 0 || i >= (int32_t)inv.w.size()) return -1;
  const WInfo& w = inv.w[i];
  if (name_out && name_cap > 0) {
    strncpy(name_out, w.name.c_str(), name_cap - 1);
    name_out[name_cap - 1] = 0;
  }
  if (shape_out)
    for (int k = 0; k < 4; ++k) shape_out[k] = w.shape[k];
  if (kind_out) *kind_out = w.kind;
  return 0;
}

static void weight_values(const WInfo& w, uint64_t seed, float bias_std, float ln_std, float* out,
                          int64_t n) {
  switch (w.kind) {
    case W_WEIGHT:
      gs_seed_normal(seed, w.name.c_str(), 0.0f, 0.02f, out, n);
      break;
    case W_BIAS:
      if (bias_std > 0) gs_seed_normal(seed, w.name.c_str(), 0.0f, bias_std, out, n);
      else memset(out, 0, n * sizeof(float));
      break;
    case W_GAMMA:
      if (ln_std > 0) gs_seed_normal(seed, w.name.c_str(), 1.0f, ln_std, out, n);
      else
        for (int64_t i = 0; i < n; ++i) out[i] = 1.0f;
      break;
    default:
      if (ln_std > 0) gs_seed_normal(seed, w.name.c_str(), 0.0f, ln_std, out, n);
      else memset(out, 0, n * sizeof(float));
  }
}

int32_t gs_mastr_weight_values(const gs_mastr_config* cfg, int32_t i, uint64_t seed,
                               float bias_std, float ln_std, float* out, int64_t n) {
  Inventory inv = make_inventory(*cfg);
  GS_REQUIRE(i >= 0 && i < (int32_t)inv.w.size(), "weight_values: index out of range");
  GS_REQUIRE(n == numel(inv.w[i]), "weight_values: numel mismatch");
  weight_values(inv.w[i], seed, bias_std, ln_std, out, n);
  return 0;
}

int32_t gs_hip_mastr_create(const gs_mastr_config* cfg, int32_t max_pairs, void** ctx_out) {
  GS_REQUIRE(cfg && ctx_out && max_pairs > 0, "mastr_create: bad arguments");
  int rc = validate_config(*cfg);
  if (rc) return rc;
  if (ensure_device()) return -2;
  Ctx* c = new Ctx();
  c->cfg = *cfg;
  c->max_pairs = max_pairs;
  c->gh = cfg->img_h / cfg->patch;
  c->gw = cfg->img_w / cfg->patch;
  c->N = c->gh * c->gw;
  c->inv = make_inventory(*cfg);
  rc = build_weights(*c);
  if (!rc) rc = build_workspace(*c);
  if (rc) {
    gs_hip_mastr_destroy(c);
    return rc;
  }
  *ctx_out = c;
  return 0;
}

void gs_hip_mastr_destroy(void* ctx) {
  if (!ctx) return;
  Ctx* c = (Ctx*)ctx;
  hipDeviceSynchronize();
  if (c->gexec) hipGraphExecDestroy(c->gexec);
  if (c->warena) hipFree(c->warena);
  if (c->wbf16) hipFree(c->wbf16);
  if (c->arena) hipFree(c->arena);
  if (c->pcbuf) hipFree(c->pcbuf);
  delete c;
}

int32_t gs_hip_mastr_init_seeded(void* ctx, uint64_t seed, float bias_std, float ln_std) {
  GS_REQUIRE(ctx, "init_seeded: null context");
  Ctx* c = (Ctx*)ctx;
  std::vector<float> buf;
  for (auto& wi : c->inv.w) {
    const int64_t n = numel(wi);
    buf.resize(n);
    weight_values(wi, seed, bias_std, ln_std, buf.data(), n);
    int rc = place_weight(*c, wi.name, buf.data(), n);
    if (rc) return rc;
  }
  return 0;
}

int32_t gs_hip_mastr_set_weight(void* ctx, const char* name, const float* host, int64_t numel_) {
  GS_REQUIRE(ctx && name && host, "set_weight: null argument");
  return place_weight(*(Ctx*)ctx, name, host, numel_);
}

int32_t gs_hip_mastr_encoder_block(void* ctx, int32_t layer, float* x, int32_t B, void* stream) {
  GS_REQUIRE(ctx && x, "encoder_block: null argument");
  Ctx* c = (Ctx*)ctx;
  GS_REQUIRE(layer >= 0 && layer < c->cfg.enc_depth, "encoder_block: layer out of range");
  GS_REQUIRE(B > 0 && B <= 2 * c->max_pairs, "encoder_block: B exceeds context capacity");
  hipStream_t s = (hipStream_t)stream;
  RC(sync_bf16(*c, s));
  return encoder_block(*c, layer, x, (int64_t)B * c->N, s);
}

int32_t gs_hip_mastr_encoder(void* ctx, const float* img, int32_t B, float* enc, void* stream) {
  GS_REQUIRE(ctx && img && enc, "encoder: null argument");
  Ctx* c = (Ctx*)ctx;
  GS_REQUIRE(B > 0 && B <= 2 * c->max_pairs, "encoder: B exceeds context capacity");
  hipStream_t s = (hipStream_t)stream;
  RC(sync_bf16(*c, s));
  RC(launch_unfold(img, B, c->cfg.img_h, c->cfg.img_w, c->cfg.patch, c->P, s));
  return encoder_from_patches(*c, B, enc, s);
}

}  // extern "C"

const gs_mastr_config* gs::mastr_ctx_config(void* ctx) { return &((Ctx*)ctx)->cfg; }

namespace {

// The pair launch sequence (encoder on both views, decoder, heads).
int pair_body(Ctx* c, const float* img1, const float* img2, int32_t B, float* pts1, float* conf1,
              float* desc1, float* pts2, float* conf2, float* desc2, hipStream_t s) {
  const gs_mastr_config& f = c->cfg;
  const int64_t Mv = (int64_t)B * c->N;
  const int64_t K = 3 * f.patch * f.patch;
  RC(launch_unfold(img1, B, f.img_h, f.img_w, f.patch, c->P, s));
  RC(launch_unfold(img2, B, f.img_h, f.img_w, f.patch, c->P + Mv * K, s));
  RC(encoder_from_patches(*c, 2 * B, c->enc, s));
  RC(decoder(*c, B, s));
  c->last_B = B;
  const float* e[2] = {c->enc, c->enc + Mv * f.enc_dim};
  const float* h6[2] = {c->hook1, c->hook1 + Mv * f.dec_dim};
  const float* h9[2] = {c->hook2, c->hook2 + Mv * f.dec_dim};
  const float* df[2] = {c->dfin, c->dfin + Mv * f.dec_dim};
  float* pts[2] = {pts1, pts2};
  float* conf[2] = {conf1, conf2};
  float* desc[2] = {desc1, desc2};
  // group the requested heads: slot v runs view hs.id[v]
  Heads hd, hl;
  const float *ge[2], *gh6[2], *gh9[2], *gdf[2], *le[2], *ldf[2];
  float *gp[2], *gc[2], *ld[2];
  for (int v = 0; v < 2; ++v) {
    if (pts[v]) {
      const int k = hd.n++;
      hd.id[k] = v + 1;
      ge[k] = e[v];
      gh6[k] = h6[v];
      gh9[k] = h9[v];
      gdf[k] = df[v];
      gp[k] = pts[v];
      gc[k] = conf[v];
    }
    if (desc[v]) {
      const int k = hl.n++;
      hl.id[k] = v + 1;
      le[k] = e[v];
      ldf[k] = df[v];
      ld[k] = desc[v];
    }
  }
  if (hd.n && f.composite == 1) RC(dpt_ref_heads(*c, hd, gdf, B, gp, gc, s));
  if (hd.n && f.composite == 0) RC(dpt_heads(*c, hd, ge, gh6, gh9, gdf, B, gp, gc, s));
  if (hl.n) RC(local_features(*c, hl, le, ldf, B, ld, s));
  return 0;
}

}  // namespace

extern "C" {

int32_t gs_hip_mastr_pair(void* ctx, const float* img1, const float* img2, int32_t B, float* pts1,
                          float* conf1, float* desc1, float* pts2, float* conf2, float* desc2,
                          void* stream) {
  GS_REQUIRE(ctx && img1 && img2, "pair: null image");
  Ctx* c = (Ctx*)ctx;
  GS_REQUIRE(B > 0 && B <= c->max_pairs, "pair: B exceeds context capacity");
  GS_REQUIRE(c->cfg.linear_layout == 0, "pair: the literal linear layout is encoder-only");
  GS_REQUIRE(!pts1 == !conf1 && !pts2 == !conf2, "pair: pts and conf must be given together");
  GS_REQUIRE(c->cfg.composite == 0 || (!desc1 && !desc2),
             "pair: composite 1 (reference stub heads) has no descriptor head");
  hipStream_t s = (hipStream_t)stream;
  RC(sync_bf16(*c, s));
  if (!c->graph_on || prof_on())
    return pair_body(c, img1, img2, B, pts1, conf1, desc1, pts2, conf2, desc2, s);
  GS_REQUIRE(s != nullptr, "pair: graph replay needs a non-null stream");
  const void* key[9] = {img1, img2, pts1, conf1, desc1, pts2, conf2, desc2, (const void*)s};
  bool hit = c->gexec != nullptr && c->gkey_B == B;
  for (int i = 0; hit && i < 9; ++i) hit = key[i] == c->gkey[i];
  if (!hit) {
    if (c->gexec) {
      GS_CHECK_HIP(hipGraphExecDestroy(c->gexec));
      c->gexec = nullptr;
    }
    GS_CHECK_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const int rc = pair_body(c, img1, img2, B, pts1, conf1, desc1, pts2, conf2, desc2, s);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(s, &g);
    if (rc) {
      if (g) hipGraphDestroy(g);
      return rc;
    }
    GS_CHECK_HIP(e);
    const hipError_t ei = hipGraphInstantiate(&c->gexec, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    GS_CHECK_HIP(ei);
    for (int i = 0; i < 9; ++i) c->gkey[i] = key[i];
    c->gkey_B = B;
  }
  c->last_B = B;
  GS_CHECK_HIP(hipGraphLaunch(c->gexec, s));
  return 0;
}

int32_t gs_hip_mastr_set_graph(void* ctx, int32_t enable) {
  GS_REQUIRE(ctx, "set_graph: null context");
  Ctx* c = (Ctx*)ctx;
  c->graph_on = enable != 0;
  if (!c->graph_on && c->gexec) {
    GS_CHECK_HIP(hipGraphExecDestroy(c->gexec));
    c->gexec = nullptr;
  }
  return 0;
}

int32_t gs_hip_mastr_pair_taps(void* ctx, int32_t B, float* enc1, float* enc2, float* dec1,
                               float* dec2, void* stream) {
  GS_REQUIRE(ctx, "pair_taps: null context");
  Ctx* c = (Ctx*)ctx;
  GS_REQUIRE(B > 0 && B <= c->last_B, "pair_taps: B exceeds the last pair call");
  hipStream_t s = (hipStream_t)stream;
  const int64_t Mv = (int64_t)c->last_B * c->N;
  const int64_t ne = (int64_t)B * c->N * c->cfg.enc_dim, nd = (int64_t)B * c->N * c->cfg.dec_dim;
  if (enc1) GS_CHECK_HIP(hipMemcpyAsync(enc1, c->enc, ne * 4, hipMemcpyDeviceToDevice, s));
  if (enc2)
    GS_CHECK_HIP(hipMemcpyAsync(enc2, c->enc + Mv * c->cfg.enc_dim, ne * 4, hipMemcpyDeviceToDevice, s));
  if (dec1) GS_CHECK_HIP(hipMemcpyAsync(dec1, c->dfin, nd * 4, hipMemcpyDeviceToDevice, s));
  if (dec2)
    GS_CHECK_HIP(hipMemcpyAsync(dec2, c->dfin + Mv * c->cfg.dec_dim, nd * 4, hipMemcpyDeviceToDevice, s));
  return 0;
}

int32_t gs_hip_mastr_frames_to_pointcloud(void* ctx, const float* frames, int32_t F,
                                          int32_t src_h, int32_t src_w, float threshold,
                                          float* out_pts, float* out_conf, int64_t capacity,
                                          int64_t* n_points, void* stream) {
  GS_REQUIRE(ctx && n_points, "frames_to_pointcloud: null argument");
  Ctx* c = (Ctx*)ctx;
  *n_points = 0;
  if (F < 2) return 0;
  GS_REQUIRE(frames, "frames_to_pointcloud: null frames");
  GS_REQUIRE(c->cfg.linear_layout == 0, "frames_to_pointcloud: needs linear_layout 0");
  GS_REQUIRE(capacity >= 0 && (capacity == 0 || (out_pts && out_conf)),
             "frames_to_pointcloud: bad output buffers");
  hipStream_t s = (hipStream_t)stream;
  const int64_t H = c->cfg.img_h, W = c->cfg.img_w;
  // point maps are at image resolution, or on the patch grid for composite 1
  const int64_t HWo = c->cfg.composite == 1 ? c->N : H * W;
  const int32_t P = F - 1;
  const int32_t Bmax = std::min(c->max_pairs, P);
  // carve the buffer
  const size_t sz_prep = align256((size_t)F * 3 * H * W * 4),
               sz_pts = align256((size_t)Bmax * HWo * 12), sz_conf = align256((size_t)Bmax * HWo * 4),
               sz_cnt = 256, sz_scr = align256((size_t)collect_points_scratch(Bmax * HWo) * 8);
  const size_t need = sz_prep + 2 * sz_pts + 2 * sz_conf + sz_cnt + sz_scr;
  if (need > c->pcbuf_size) {
    if (c->pcbuf) {
      GS_CHECK_HIP(hipDeviceSynchronize());
      GS_CHECK_HIP(hipFree(c->pcbuf));
      c->pcbuf = nullptr;
      c->pcbuf_size = 0;
    }
    GS_CHECK_HIP(hipMalloc(&c->pcbuf, need));
    c->pcbuf_size = need;
  }
  char* cur = c->pcbuf;
  float* prep = (float*)cur;
  cur += sz_prep;
  float* pts1 = (float*)cur;
  cur += sz_pts;
  float* pts2 = (float*)cur;
  cur += sz_pts;
  float* conf1 = (float*)cur;
  cur += sz_conf;
  float* conf2 = (float*)cur;
  cur += sz_conf;
  int64_t* counter = (int64_t*)cur;
  cur += sz_cnt;
  int64_t* scratch = (int64_t*)cur;

  RC(launch_fill_i64(counter, 1, 0, s));
  RC(launch_image_prep(frames, F, src_h, src_w, 3, (int32_t)H, (int32_t)W, true, true, true, prep,
                       s));
  RC(sync_bf16(*c, s));
  for (int32_t p0 = 0; p0 < P; p0 += Bmax) {
    const int32_t Bc = std::min(Bmax, P - p0);
    const bool last = p0 + Bc == P;
    RC(pair_body(c, prep + (int64_t)p0 * 3 * H * W, prep + (int64_t)(p0 + 1) * 3 * H * W, Bc,
                 pts1, conf1, nullptr, last ? pts2 : nullptr, last ? conf2 : nullptr, nullptr, s));
    RC(launch_collect_points(pts1, conf1, (int64_t)Bc * HWo, threshold, out_pts, out_conf,
                             capacity, counter, scratch, s));
    if (last)
      RC(launch_collect_points(pts2 + (int64_t)(Bc - 1) * HWo * 3,
                               conf2 + (int64_t)(Bc - 1) * HWo, HWo, threshold, out_pts, out_conf,
                               capacity, counter, scratch, s));
  }
  int64_t n = 0;
  GS_CHECK_HIP(hipMemcpyAsync(&n, counter, sizeof(n), hipMemcpyDeviceToHost, s));
  GS_CHECK_HIP(hipStreamSynchronize(s));
  *n_points = n;
  return 0;
}

}  // extern "C"
