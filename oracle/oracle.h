/*
 * oracle.h -- CPU restatement of crystal-gausplat's MASt3R inference arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it. The product library (libgsplat_hip.so) never links or calls it.
 *
 * Arithmetic contract (what "restatement" means here):
 *   - fp32 everywhere, sums accumulated sequentially in the reference's loop
 *     order, built with -ffp-contract=off and no fast-math, libm expf / tanhf /
 *     sqrtf / cosf / sinf / powf (Crystal's Math.* on Float32 lowers to the
 *     same libm calls).
 *   - Some loops are blocked or vectorised ACROSS independent output elements;
 *     the per-element sequence of fp32 operations is unchanged, so results are
 *     bit-identical to the literal reference loop (tests assert this against
 *     the *_naive variants).
 *
 * Parity pinning: see the header of oracle.cpp for which check pins which
 * function. Functions marked "parity unpinned" there have no independent pin.
 */
#ifndef GS_ORACLE_H
#define GS_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- threading ---------------------------------------------------------- */
void orc_set_threads(int32_t n);           /* 0 = all OpenMP threads */
int32_t orc_get_threads(void);

/* ---- primitives --------------------------------------------------------- */
/* y[M,N] = x[M,K] . W + b.  layout 0: W is [N,K] (y = x W^T, the reference GPU
 * path and MASt3R semantics).  layout 1: W buffer read as [K,N] (the reference
 * CPU path's literal indexing b_d[kk*n+j], src/nn/linear.cr:194).  b nullable. */
void orc_linear(const float* x, int64_t M, int32_t K, const float* W,
                const float* b, int32_t N, float* y, int32_t layout);
void orc_linear_naive(const float* x, int64_t M, int32_t K, const float* W,
                      const float* b, int32_t N, float* y, int32_t layout);

void orc_layernorm(const float* x, int64_t rows, int32_t D, const float* gamma,
                   const float* beta, float eps, float* y);
void orc_gelu(const float* x, int64_t n, float* y);
void orc_relu(const float* x, int64_t n, float* y);
void orc_add(const float* a, const float* b, int64_t n, float* y);

/* q [B,H,Nq,hd], k,v [B,H,Nkv,hd] -> o [B,H,Nq,hd] */
void orc_sdpa(const float* q, const float* k, const float* v, float* o,
              int32_t B, int32_t H, int32_t Nq, int32_t Nkv, int32_t hd,
              float scale);

void orc_sdpa_naive(const float* q, const float* k, const float* v, float* o,
                    int32_t B, int32_t H, int32_t Nq, int32_t Nkv, int32_t hd,
                    float scale);
/* 1: composites use the literal reference loops (orc_linear_naive,
 * orc_sdpa_naive, orc_conv2d_naive) -- the CPU-baseline configuration. */
void orc_set_naive(int32_t on);
/* Test-only: plant composition mistake m in the composites (0 = none):
 * 1 cross-attention memory = the other view's decoder_embed output, fixed;
 * 2 norm_y dropped; 3 no RoPE on the cross-attention q / k; 4 local-feature
 * concat in dec | enc order; 5 norm2 / norm3 roles swapped. Used only to
 * show that the composition pins fail on each. */
void orc_set_mutation(int32_t m);

/* RoPE2D tables: cos/sin[pos][j], j < hd/4, pos < max_pos. */
void orc_rope_table(int32_t max_pos, int32_t hd, float base, float* cos_t,
                    float* sin_t);
/* In-place 2D RoPE on t [B, N, H*hd] (token-major, heads interleaved).
 * Token n sits at (y, x) = (n / grid_w, n % grid_w). */
void orc_rope2d(float* t, int32_t B, int32_t N, int32_t H, int32_t hd,
                int32_t grid_w, float base);
/* Reference token-level RoPE (src/mastr/encoder_v2.cr:180-258), generalised to
 * an explicit (grid_h, grid_w); x [B, N, D], heads of hd. */
void orc_rope_ref_token(const float* x, float* y, int32_t B, int32_t grid_h,
                        int32_t grid_w, int32_t D, int32_t H, float base);

/* NCHW image [B,C,H,W] -> patches [B, (H/p)*(W/p), C*p*p] in (c,i,j) order. */
void orc_unfold(const float* img, int32_t B, int32_t C, int32_t H, int32_t W,
                int32_t p, float* out);

/* NHWC x [B,H,W,Cin], OIHW w [Cout,Cin,k,k] -> y [B,Ho,Wo,Cout]. b nullable. */
void orc_conv2d(const float* x, int32_t B, int32_t H, int32_t W, int32_t Cin,
                const float* w, const float* b, int32_t Cout, int32_t k,
                int32_t stride, int32_t pad, float* y);
void orc_conv2d_naive(const float* x, int32_t B, int32_t H, int32_t W,
                      int32_t Cin, const float* w, const float* b, int32_t Cout,
                      int32_t k, int32_t stride, int32_t pad, float* y);
/* kh x kw kernels: OIHW w [Cout,Cin,kh,kw], Ho = (H+2pad-kh)/stride+1,
 * Wo = (W+2pad-kw)/stride+1; orc_conv2d is the kh == kw == k case. */
void orc_conv2d_hw(const float* x, int32_t B, int32_t H, int32_t W, int32_t Cin,
                   const float* w, const float* b, int32_t Cout, int32_t kh,
                   int32_t kw, int32_t stride, int32_t pad, float* y);
void orc_conv2d_hw_naive(const float* x, int32_t B, int32_t H, int32_t W,
                         int32_t Cin, const float* w, const float* b,
                         int32_t Cout, int32_t kh, int32_t kw, int32_t stride,
                         int32_t pad, float* y);
/* ConvTranspose2d with kernel == stride, no padding. w [Cin,Cout,k,k]. */
void orc_conv_transpose(const float* x, int32_t B, int32_t H, int32_t W,
                        int32_t Cin, const float* w, const float* b,
                        int32_t Cout, int32_t k, float* y);
/* Bilinear x2, align_corners=True, NHWC. */
void orc_upsample2x(const float* x, int32_t B, int32_t H, int32_t W, int32_t C,
                    float* y);
/* Pixel-shuffle of the local-feature MLP output: f [B, h*w, Cf] with
 * Cf >= C*r*r -> desc [B, h*r, w*r, C] NHWC, desc[c] at (r*y+i, r*x+j) =
 * f[token (y,x)][c*r*r + i*r + j]. */
void orc_pixel_shuffle(const float* f, int32_t B, int32_t h, int32_t w,
                       int32_t Cf, int32_t r, int32_t C, float* desc);

/* ---- caller-side image and point-cloud passes --------------------------- */
/* resize_image (src/mastr/inference.cr:330-374): bilinear, align-corners
 * mapping sy = ty*(sh-1)/(th-1) in fp32, x0/y0 clamped to [0, s-2].
 * src [sh, sw, C] -> dst [th, tw, C]; needs sh, sw, th, tw >= 2. */
void orc_resize_image(const float* src, int32_t sh, int32_t sw, int32_t C,
                      int32_t th, int32_t tw, float* dst);
/* preprocess_image (src/mastr/inference.cr:193-229): [B,H,W,3] in [0,1] ->
 * [B,3,H,W], (v - mean[c]) / std[c] with the ImageNet mean / std. */
void orc_preprocess_image(const float* src, int32_t B, int32_t H, int32_t W,
                          float* dst);
/* collect_points (src/mastr/inference.cr:296-328): the points whose
 * confidence is > threshold, in element order. pts [n,3], conf [n] ->
 * out_pts [k,3], out_conf [k]; returns k. */
int64_t orc_collect_points(const float* pts, const float* conf, int64_t n,
                           float threshold, float* out_pts, float* out_conf);

/* ---- composites --------------------------------------------------------- */
typedef struct orc_config {
  int32_t img_h, img_w, patch;
  int32_t enc_dim, enc_depth, enc_heads, enc_mlp;
  int32_t dec_dim, dec_depth, dec_heads, dec_mlp;
  int32_t dpt_feat;          /* 256 */
  int32_t dpt_dims[4];       /* act_postprocess widths 96,192,384,768 */
  int32_t dpt_hooks[4];      /* 0, 6, 9, 12 */
  int32_t head_mid;          /* 128 */
  int32_t lf_hidden;         /* 7168 */
  int32_t desc_dim;          /* 24 */
  float ln_eps;              /* 1e-6 */
  float rope_base;           /* 100 */
  int32_t linear_layout;     /* 0 = x W^T, 1 = reference CPU literal */
  int32_t rope_mode;         /* 0 none, 1 per-attention q/k 2D, 2 ref-token */
  int32_t composite;         /* 0 MASt3R composition; 1 the reference's
                                literal forward_pair (own-view decoder
                                memory, stub DPT on the patch grid, sigmoid
                                confidence, no descriptors) */
} orc_config;

/* Weights are fetched by name through a callback (arrays owned by caller). */
typedef const float* (*orc_weight_fn)(const char* name, void* user);

/* One encoder block in place on x [B, N, D]; prefix e.g. "enc_blocks.0". */
int32_t orc_encoder_block(const orc_config* cfg, const char* prefix,
                          orc_weight_fn wf, void* user, float* x, int32_t B,
                          int32_t grid_h, int32_t grid_w);
/* One decoder block (src/mastr/decoder_v2.cr:47-63) in place on x [B,N,D];
 * mem [B,N,D] is the cross-attention memory; prefix e.g. "dec_blocks.0". */
int32_t orc_decoder_block(const orc_config* cfg, const char* prefix,
                          orc_weight_fn wf, void* user, float* x,
                          const float* mem, int32_t B, int32_t grid_h,
                          int32_t grid_w);
/* Local-feature head: fc2(GELU(fc1(concat(enc, dec)))) over tokens, then the
 * pixel shuffle by `patch`, channels [0, desc_dim): enc [B,N,enc_dim],
 * dec [B,N,dec_dim] (the dec_norm output) -> desc [B,gh*patch,gw*patch,
 * desc_dim]; prefix e.g. "downstream_head1". */
int32_t orc_local_features(const orc_config* cfg, orc_weight_fn wf, void* user,
                           const char* prefix, const float* enc,
                           const float* dec, int32_t B, int32_t gh, int32_t gw,
                           float* desc);
/* Full encoder: img [B,3,H,W] -> enc [B, N, enc_dim] (after enc_norm). */
int32_t orc_encoder(const orc_config* cfg, orc_weight_fn wf, void* user,
                    const float* img, int32_t B, float* enc);
/* Full two-view pair: outputs NHWC per view (composite 1: pts / conf on the
 * patch grid, desc must be NULL; returns -1 otherwise). */
int32_t orc_mastr_pair(const orc_config* cfg, orc_weight_fn wf, void* user,
                       const float* img1, const float* img2, int32_t B,
                       float* pts1, float* conf1, float* desc1, float* pts2,
                       float* conf2, float* desc2);
/* One full DPT head (composite 0) on its four hooks: hooks[0] [B,N,enc_dim],
 * hooks[1..3] [B,N,dec_dim] on the gh x gw grid; prefix e.g.
 * "downstream_head1"; pts [B,H,W,3], conf [B,H,W,1] at 16x the grid. */
int32_t orc_dpt_head(const orc_config* cfg, orc_weight_fn wf, void* user,
                     const char* prefix, const float* const hooks[4], int32_t B,
                     int32_t gh, int32_t gw, float* pts, float* conf);
/* Intermediate taps for debugging the pair path (all nullable):
 * enc1/enc2 [B,N,enc_dim]; dec1/dec2 [B,N,dec_dim] = dec_norm(d^depth). */
int32_t orc_mastr_pair_taps(const orc_config* cfg, orc_weight_fn wf,
                            void* user, const float* img1, const float* img2,
                            int32_t B, float* enc1, float* enc2, float* dec1,
                            float* dec2);

#ifdef __cplusplus
}
#endif
#endif
