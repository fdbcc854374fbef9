// Internal declarations shared by the HIP kernels, the C-ABI shim and the
// MASt3R orchestration. Not part of the public ABI (include/gs_hip.h is).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

struct gs_mastr_config;

namespace gs {

// Native 4-wide float vector for kernels (HIP's float4 struct is copied via
// memcpy, which keeps register arrays of it out of VGPRs).
typedef float fx4 __attribute__((ext_vector_type(4)));
__host__ __device__ inline fx4 mk4(float a, float b, float c, float d) {
  fx4 r = {a, b, c, d};
  return r;
}

// ---- error state (thread-local last error, see gs_hip_last_error) ----------
void set_error(const std::string& msg);
const char* last_error();
hipStream_t default_stream();  // library stream; created by gs_init_device
int ensure_device();           // 0 ok; lazily runs gs_init_device

#define GS_CHECK_HIP(expr)                                                    \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess) {                                                   \
      ::gs::set_error(std::string(#expr " failed: ") + hipGetErrorString(e_)); \
      return -3;                                                              \
    }                                                                         \
  } while (0)

#define GS_REQUIRE(cond, msg)       \
  do {                              \
    if (!(cond)) {                  \
      ::gs::set_error(msg);         \
      return -1;                    \
    }                               \
  } while (0)

// ---- per-kernel timing (gs_hip_profile_*) ------------------------------------
// When enabled, launchers bracket each kernel with HIP events on its stream and
// record (kernel name, algorithmic flops, algorithmic HBM bytes).
bool prof_on();
bool prof_per_shape();
hipEvent_t prof_start(hipStream_t s);
void prof_stop(hipStream_t s, hipEvent_t start, const char* kernel, double flops,
               double bytes);

// Sum over the 64 lanes of a wavefront (butterfly; every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// ---- GEMM ------------------------------------------------------------------
// C[M,N] = A[M,K] . B (+ epilogue). One GEMM problem of a (possibly grouped)
// launch. All pointers are device pointers.
// A_PLAIN_H: plain rows of a bf16 A (the bf16 kernels only; lda in elements)
// A_LN: plain rows with the LayerNorm apply step fused into the load:
// a = (x - mean[row]) * inv_std[row] * gamma[k] + beta[k], the same
// expression as the LayerNorm kernel (bit-identical operands), row statistics
// from its stats pass.
// A_CONV_H: implicit conv on a bf16 NHWC input (the bf16 kernels only).
enum ALoad : int { A_PLAIN = 0, A_CONCAT = 1, A_CONV = 2, A_PLAIN_H = 3, A_LN = 4, A_CONV_H = 5 };
enum BLayout : int { B_NT = 0, B_NN = 1 };

enum EpiFlags : int {
  EPI_BIAS = 1,
  EPI_GELU = 2,
  EPI_RELU = 4,
  EPI_RES1 = 8,      // v = v + R1
  EPI_RES2 = 16,     // v = R2 + v (applied after RES1)
  EPI_ROPE = 32,     // RoPE on columns [0, rope_ncols)
  EPI_SCATTER = 64,  // sub-pixel scatter store (ConvT / pixel shuffle)
  EPI_DUAL = 128,    // also store the result to C2 (same ldc)
  EPI_BF16OUT = 256, // C holds bf16 (ldc in elements; with SCATTER the scattered store); not with DUAL
  EPI_LNOUT = 512,   // also the LayerNorm of every output row into lnout (see GemmArgs)
  EPI_DUAL_RELU_H = 1024,  // with EPI_DUAL: C2 holds bf16 and receives bf16(max(v, 0))
};

struct GemmArgs {
  const float* A;   // plain / concat first source / conv input (NHWC)
  int64_t lda;
  const float* A2;  // concat second source
  int64_t lda2;
  int32_t K1;       // concat split (multiple of 32)
  // implicit convolution (A_CONV): input [Bimg, cH, cW, cCin], kernel
  // ck (rows) x ckw (columns), stride cs, pad cp, output grid cHo x cWo;
  // K = ck*ckw*cCin, k index = (kh*ckw + kw)*cCin + ic
  int32_t cH, cW, cCin, ck, cs, cp, cHo, cWo, ckw;
  const float* B;   // NT: B[n*ldb + k]; NN: B[k*ldb + n]
  const void* Bh;   // bf16 copy of B (NT layout, same ldb) for the bf16 kernels;
                    // for the bf16x6 kernel with bh_plane > 0: plane 0 of the
                    // three-term bf16 split of B, plane t at Bh + t * bh_plane
  int64_t bh_plane; // elements between the split planes (0: split B on the fly)
  int64_t ldb;
  float* C;
  int64_t ldc;
  float* C2;        // second destination of EPI_DUAL
  const float* bias;
  const float* R1;
  int64_t ldr1;
  const float* R2;
  int64_t ldr2;
  int32_t M, N, K;
  int32_t flags;
  // RoPE epilogue: columns [0, rope_ncols) hold 64-wide heads; row m is token
  // (m % tok_per_img) of a grid with grid_w columns; tables [pos][16].
  const float* rope_cos;
  const float* rope_sin;
  int32_t rope_ncols, tok_per_img, grid_w;
  // A_LN: per-row (mean, inv_std) pairs and the LayerNorm's gamma / beta [K]
  const float* ln_stats;
  const float* ln_g;
  const float* ln_b;
  // scatter epilogue: row m = (img, y, x) on a sc_gh x sc_gw grid; column
  // n = (i*sc_r + j)*sc_C + c -> C[((img*sc_gh*sc_r + y*sc_r + i)*sc_gw*sc_r
  // + x*sc_r + j)*sc_C + c]; columns with c >= sc_Cout are dropped.
  int32_t sc_r, sc_C, sc_gh, sc_gw, sc_Cout;
  // split-K partials [ksplit][M][N] of this group (set by launch_gemm)
  float* part;
  // EPI_LNOUT: once a row of C is final, its LayerNorm over the N columns,
  // lnout = (c - mean) * inv_std * lnout_g + lnout_b (same arithmetic and
  // order as the LayerNorm kernel), rows of N floats. Split launches do it in
  // the reduce pass; otherwise launch_gemm runs the LayerNorm kernel after
  // the GEMM. Bias / residual epilogues only, N % 4 == 0, N <= 4096, ldc == N.
  float* lnout;
  const float* lnout_g;
  const float* lnout_b;
  float lnout_eps;
};

constexpr int kMaxGroups = 2;
struct GemmBatch {
  GemmArgs g[kMaxGroups];
  int32_t ngroups;
  // Optional split-K scratch (floats). When it is given and the launch would
  // leave most CUs idle, launch_gemm splits K into ksplit contiguous ranges
  // whose partial tiles a second kernel sums in a fixed order (so results are
  // deterministic) before the epilogue.
  float* part_ws = nullptr;
  int64_t part_ws_elems = 0;
  int32_t ksplit = 0;  // 0: chosen by launch_gemm; > 0: requested split (validated)
  // fp32 kernel: 0 chosen by launch_gemm; requested (validated): 1 register-staged,
  // 2 direct-to-LDS, 3 bf16x6 (fp32-accurate products on bf16 matrix cores)
  int32_t kernel = 0;
  // set by launch_gemm for the tile-phase launches of the 256 x 128 fp32
  // kernel (0: one launch covers every tile): workgroup b runs tile
  // (b % 8) * tphase_q + tphase_base + b / 8 of the group's XCD-major order
  int32_t tphase_q = 0, tphase_base = 0;
};

// Launch a grouped GEMM (all groups must share the loader / layout kinds).
// bf16: bf16-input / fp32-accumulate MFMA on the groups' Bh weight copies.
int launch_gemm(const GemmBatch& b, int aload, int blayout, bool a_relu,
                hipStream_t s, bool bf16 = false);
int check_gemm(const GemmArgs& a, int aload, int blayout, bool bf16 = false);

// ---- attention -----------------------------------------------------------------
struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  int64_t q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn, o_sb, o_sh, o_sn;
  int32_t B, H, Nq, Nkv;
  float scale;
  int32_t o_bf16 = 0;  // o holds bf16 (strides in elements); bf16 kernel only
  int32_t in_bf16 = 0; // q, k, v hold bf16 (strides in elements); bf16 kernel only
};
struct AttnBatch {
  AttnArgs g[kMaxGroups];
  int32_t ngroups;
  // Optional scratch (floats). When it is given and the launch would leave
  // most CUs idle, launch_attention splits the keys into kv_split ranges of
  // kv_chunk keys; a second kernel merges the ranges' softmax states in range
  // order (deterministic).
  float* part_ws = nullptr;
  int64_t part_ws_elems = 0;
  int32_t kv_split = 0;  // 0: chosen by launch_attention; > 0: requested ranges
  int32_t kv_chunk = 0;
};
// prec: 0 fp32 MFMA, 1 bf16-input, 2 bf16x6 split products (fp32 accuracy;
// launches that split the keys use the fp32 kernel)
int launch_attention(const AttnBatch& b, hipStream_t s, int prec = 0);
// Scratch (floats) that lets launch_attention split the keys of this launch
// as far as its cost model may choose; 0 when the launch never splits.
int64_t attention_split_elems(const AttnBatch& b, int prec = 0);

// ---- LayerNorm -----------------------------------------------------------------
struct LnArgs {
  const float* x;
  const float* gamma;
  const float* beta;
  float* y;
  int64_t rows;
  int32_t D;
  float eps;
  int32_t y_bf16 = 0;  // y holds bf16
  float* stats = nullptr;  // optional (mean, inv_std) per row; y may then be null
};
struct LnBatch {
  LnArgs g[kMaxGroups];
  int32_t ngroups;
};
int launch_layernorm(const LnBatch& b, hipStream_t s);

// ---- small kernels -----------------------------------------------------------
int launch_unfold(const float* img, int32_t B, int32_t H, int32_t W, int32_t p,
                  float* out, hipStream_t s);
// out_bf16: y holds bf16 (for a bf16 conv that reads it, A_CONV_H)
int launch_upsample2x(const float* x, int32_t B, int32_t H, int32_t W,
                      int32_t C, float* y, hipStream_t s, bool out_bf16 = false,
                      bool in_bf16 = false);
int launch_rope2d(float* t, int32_t B, int32_t N, int32_t H, int64_t ld,
                  int32_t grid_w, const float* cos_t, const float* sin_t,
                  hipStream_t s);
// Token-level RoPE of the reference; tables cos/sin [max_pos][hd/2].
int launch_rope_ref_token(const float* x, float* y, int32_t B, int32_t gh,
                          int32_t gw, int32_t D, int32_t H, const float* cos_t,
                          const float* sin_t, int32_t max_pos, hipStream_t s);
// conv 1x1 Cin->4 + split: pts [P,3] = y[0..2], conf [P] = 1 + exp(y[3]).
int launch_head_out(const float* x, int64_t P, int32_t Cin, const float* w, const float* b,
                    float* pts, float* conf, bool sigmoid, hipStream_t s, bool in_bf16 = false);

// Weight re-layouts (device): OIHW -> OHWI; ConvTranspose [Cin,Cout,k,k] ->
// [(i*k+j)*Cout + oc][Cin] with the bias expanded to k*k*Cout columns.
int launch_oihw_to_ohwi(const float* w, int32_t Cout, int32_t Cin, int32_t k,
                        float* out, hipStream_t s);
int launch_convt_relayout(const float* w, const float* b, int32_t Cin,
                          int32_t Cout, int32_t k, float* wout, float* bout,
                          hipStream_t s);

// fp32 -> bf16 (round to nearest even), n elements.
int launch_f32_to_bf16(const float* in, void* out, int64_t n, hipStream_t s);
// Exact three-term bf16 split x = x0 + x1 + x2 of n floats: plane t at
// out + t * plane (bf16 elements), plane >= n.
int launch_f32_to_bf16x3(const float* in, void* out, int64_t n, int64_t plane, hipStream_t s);

// RoPE tables for 64-wide heads: cos/sin [max_pos][16], host computed.
void rope_table_host(int32_t max_pos, float base, float* cos_t, float* sin_t);
// Reference token-level RoPE tables: cos/sin [max_pos][hd/2] of
// pos * 1/base^(2i/hd) (src/mastr/encoder_v2.cr:165-176).
void rope_ref_table_host(int32_t max_pos, int32_t hd, float base, float* cos_t,
                         float* sin_t);

// Caller-side passes (pointcloud.hip). image_prep: F frames [sh,sw,C] ->
// [F,th,tw,C] (resize only) or [F,3,th,tw] (normalize, with or without
// resize). collect_points: appends the points with conf > thr at *counter
// (device int64, advanced by the selected count; positions >= cap are not
// written); scratch holds collect_points_scratch(n) int64.
int launch_image_prep(const float* src, int32_t F, int32_t sh, int32_t sw, int32_t C,
                      int32_t th, int32_t tw, bool resize, bool normalize, bool nchw,
                      float* dst, hipStream_t s);
int64_t collect_points_scratch(int64_t n);
int launch_collect_points(const float* pts, const float* conf, int64_t n, float thr,
                          float* out_pts, float* out_conf, int64_t cap, int64_t* counter,
                          int64_t* scratch, hipStream_t s);
int launch_fill_i64(int64_t* p, int64_t n, int64_t v, hipStream_t s);

// General-shape kernels of the op-level entry points (general.hip): attention
// for any head_dim >= 1 and any strides / alignment; LayerNorm of any
// width and alignment; a zero-padded, possibly transposing copy
// dst[r*cp + c] = c < cols ? src[r*s_row + c*s_col] : 0; and a convolution
// weight (OIHW layout 0 / OHWI layout 1) of kh x kw taps to OHWI with Cin
// padded to cp.
int launch_attention_general(const AttnArgs& a, int32_t hd, hipStream_t s);
int launch_layernorm_rows(const LnArgs& a, hipStream_t s);
int launch_stage(const float* src, int64_t rows, int64_t cols, int64_t s_row, int64_t s_col,
                 float* dst, int64_t cp, hipStream_t s);
int launch_conv_weight_stage(const float* w, int32_t Cout, int32_t Cin, int32_t kh, int32_t kw,
                             int32_t layout, int32_t cp, float* out, hipStream_t s);

// Configuration of a MASt3R context created by gs_hip_mastr_create.
const ::gs_mastr_config* mastr_ctx_config(void* ctx);

}  // namespace gs
