/*
 * gs_hip.h -- C ABI of libgsplat_hip.so, the MI355X (gfx950) backend that
 * replaces crystal-gausplat's Metal bridge for the MASt3R inference path.
 *
 * Three groups of entry points:
 *
 *  1. Kept gs_* buffer/device symbols, same C signatures as the Metal bridge
 *     exports (src/metal/bridge.mm:362-482), declared on the Crystal side in
 *     `lib MetalFFI` (src/core/buffer.cr:214-222) and `lib MetalDeviceFFI`
 *     (src/metal/device.cr:206-251). Buffers are explicit device allocations;
 *     gs_buffer_contents returns a DEVICE pointer (not host-dereferenceable).
 *     The pipeline / command-buffer / encoder symbols of the bridge
 *     (gs_create_pipeline*, gs_create_command_buffer, gs_commit*,
 *     gs_create_compute_encoder, gs_encoder_*) have no counterpart: kernels are
 *     precompiled for gfx950 and are reached through the op-level entry points.
 *
 *  2. Op-level entry points: one per NN::GPUOps operation on the path
 *     (src/nn/gpu_ops.cr), plus the operations the reference runs on the CPU
 *     between GPU calls (RoPE, resampling, head split).
 *
 *  3. Graph-level entry points: a MASt3R context holding device weights and
 *     workspaces, running whole encoder / pair forwards as one launch
 *     sequence on a stream (MASt3RInference#forward_pair,
 *     src/mastr/inference.cr:92-115).
 *
 * Conventions (new): every gs_hip_* call returns int32 status, 0 = ok, < 0 =
 * error, with gs_hip_last_error() describing the last failure of the calling
 * thread. Pointers passed to gs_hip_* compute calls are device pointers
 * (hipMalloc'd or gs_buffer_contents) unless named host_*. `stream` is a
 * hipStream_t; NULL is HIP's default (null) stream, as in the HIP runtime.
 * The library's own stream, which the kept gs_buffer_* copies use, is the
 * one gs_get_command_queue returns; a caller mirroring the reference's single
 * queue passes that. All compute calls are asynchronous on their stream and
 * launch nothing before their host-side shape checks pass. All tensors are
 * fp32, row-major, contiguous unless strides are given.
 */
#ifndef GS_HIP_H
#define GS_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* 1. Kept buffer / device symbols                                           */
/* ------------------------------------------------------------------------ */

/* src/metal/bridge.mm:363 (gs_create_buffer). storage_mode is accepted and
 * ignored: every buffer is device memory. Returns NULL on failure. */
void* gs_create_buffer(int64_t size, int32_t storage_mode);
/* src/metal/bridge.mm:367. Synchronises the library stream, then frees. */
void gs_release_buffer(void* handle);
/* src/metal/bridge.mm:371. Device pointer of the buffer. */
void* gs_buffer_contents(void* handle);
/* src/metal/bridge.mm:375 / 379. Host <-> device copy, synchronous. */
void gs_buffer_write(void* handle, void* data, int64_t size);
void gs_buffer_read(void* handle, void* dest, int64_t size);
/* src/metal/bridge.mm:383. No-op (no managed storage). */
void gs_buffer_sync(void* handle);
/* src/metal/bridge.mm:387. Device-to-device copy on the library stream. */
void gs_buffer_copy(void* src_handle, void* dst_handle, int64_t size);

/* Asynchronous host <-> device copies (no bridge counterpart: Metal's shared
 * storage needed none; discrete device memory needs explicit copies): size
 * bytes between host memory and the buffer at byte offset,
 * enqueued on `stream` (NULL = HIP default stream). The host memory must stay
 * valid until the stream reaches the copy; pinned memory from gs_host_alloc
 * makes the copy truly asynchronous. Return 0, or -1 (bad handle / range). */
int32_t gs_buffer_write_async(void* handle, const void* host, int64_t size,
                              int64_t offset, void* stream);
int32_t gs_buffer_read_async(void* handle, void* host, int64_t size,
                             int64_t offset, void* stream);
/* Pinned (page-locked) host memory for the async copies; NULL on failure. */
void* gs_host_alloc(int64_t size);
void gs_host_free(void* ptr);
/* Wait for `stream` (NULL = HIP default stream). */
int32_t gs_stream_synchronize(void* stream);

/* src/metal/bridge.mm:392. 0 = ok, -1 = no device, -2 = stream failure. */
int32_t gs_init_device(void);
/* src/metal/bridge.mm:396 / 400. Opaque device handle / the hipStream_t. */
void* gs_get_device(void);
void* gs_get_command_queue(void);
/* src/metal/bridge.mm:404. hipStreamSynchronize on the library stream. */
void gs_synchronize(void);
/* src/metal/bridge.mm:408-422. */
const char* gs_device_name(void);
int32_t gs_max_threads_per_threadgroup(void);
int64_t gs_recommended_working_set_size(void);
int32_t gs_has_unified_memory(void);

/* ------------------------------------------------------------------------ */
/* Errors                                                                    */
/* ------------------------------------------------------------------------ */
const char* gs_hip_last_error(void);

/* ------------------------------------------------------------------------ */
/* Seeded synthetic data (host side, shared by tests and the context)        */
/* ------------------------------------------------------------------------ */
/* SplitMix64 stream keyed by (seed, FNV-1a(name)); normal by Box-Muller from
 * 24-bit uniforms; values rounded to fp32. Deterministic across hosts. */
void gs_seed_normal(uint64_t seed, const char* name, float mean, float std,
                    float* host_out, int64_t n);
void gs_seed_uniform(uint64_t seed, const char* name, float lo, float hi,
                     float* host_out, int64_t n);

/* ------------------------------------------------------------------------ */
/* 2. Op-level entry points                                                  */
/* ------------------------------------------------------------------------ */

/* Epilogue flags for gs_hip_linear. */
#define GS_EPI_GELU 1     /* y = gelu_tanh(x.W + b)                          */
#define GS_EPI_RESIDUAL 2 /* y = residual + (x.W + b)                        */
#define GS_EPI_RELU 4     /* y = max(x.W + b, 0)                             */
#define GS_EPI_BF16 8     /* bf16-input / fp32-accumulate MFMA (w_layout 0)  */
#define GS_EPI_F32X6 16   /* fp32 through bf16 matrix cores: exact three-term
                             bf16 split of both operands, six term products,
                             fp32 accumulate (fp32-level accuracy; w_layout 0) */

/* NN::GPUOps.linear_forward (src/nn/gpu_ops.cr:39-78) plus the bias add the
 * reference does on the CPU (src/nn/linear.cr:206-230).
 * y[M,N] = x[M,K] . W (+ b) with the epilogue above.
 * w_layout 0: W is [N,K] (y = x W^T, the GPU path's semantics);
 * w_layout 1: W buffer read as [K,N] (the reference CPU path's literal
 * indexing, src/nn/linear.cr:194). Any M >= 0, K >= 1, N >= 1 (the reference's
 * linear_forward takes any width; linear_forward_simple serves in or out
 * below 64, nn.metal:84-110): K % 32 == 0 with 16-byte aligned x and W runs
 * on them directly; other shapes on zero-padded copies of x and W in
 * stream-ordered scratch (allocated and released on `stream`). b, residual
 * nullable. residual may alias y. */
int32_t gs_hip_linear(const float* x, const float* w, const float* b, float* y,
                      int64_t M, int32_t K, int32_t N, int32_t w_layout,
                      int32_t epilogue, const float* residual, void* stream);

/* NN::GPUOps.layernorm_forward (src/nn/gpu_ops.cr:114-138), the arithmetic of
 * LayerNorm#forward_cpu (src/nn/layernorm.cr:192-240). Any D >= 1: one
 * wavefront per row for 16-byte aligned rows with D % 4 == 0 and D <= 4096,
 * one workgroup per row otherwise. */
int32_t gs_hip_layernorm(const float* x, const float* gamma, const float* beta,
                         float* y, int64_t rows, int32_t D, float eps,
                         void* stream);

/* NN::GPUOps.fused_attention (src/nn/gpu_ops.cr:200-227) generalised to
 * cross-attention with Nq != Nkv (the CPU path's semantics,
 * src/nn/attention.cr:215-325). Any head_dim >= 1, as the reference (its own
 * spec runs 16, spec/nn/attention_spec.cr:49-58): head_dim 64 with 16-byte
 * aligned rows (pointers and strides multiples of 4 floats) runs on the MFMA
 * flash kernel, anything else on a general kernel (one wavefront per query,
 * K / V tiles in LDS, expf softmax; head dims beyond 128 in chunks of 128,
 * accumulated in the output row). Element (b,h,n,d) of q
 * is at q[b*q_sb + h*q_sh + n*q_sn + d]; likewise for k, v, o. The
 * reference layout [B,H,N,64] is q_sb = H*N*64, q_sh = N*64, q_sn = 64;
 * token-major [B,N,H*64] is q_sb = N*H*64, q_sh = 64, q_sn = H*64. */
int32_t gs_hip_attention(const float* q, const float* k, const float* v,
                         float* o, int32_t B, int32_t H, int32_t Nq,
                         int32_t Nkv, int32_t head_dim, float scale,
                         int64_t q_sb, int64_t q_sh, int64_t q_sn,
                         int64_t k_sb, int64_t k_sh, int64_t k_sn,
                         int64_t v_sb, int64_t v_sh, int64_t v_sn,
                         int64_t o_sb, int64_t o_sh, int64_t o_sn,
                         void* stream);

/* gs_hip_attention with a choice of arithmetic, as gs_hip_linear's epilogue
 * flags choose it for the linears: precision 0 = fp32 MFMA (gs_hip_attention
 * itself); 1 = the bf16-input / fp32-accumulate variant (q, k, v and the
 * softmax probabilities rounded to bf16; the north star's optional bf16
 * path); 2 = fp32 through bf16x6 split products (fp32-level accuracy;
 * launches that split the keys run the fp32 kernel). Precisions 1 and 2 need
 * head_dim 64 and 16-byte aligned rows. */
int32_t gs_hip_attention_prec(const float* q, const float* k, const float* v,
                              float* o, int32_t B, int32_t H, int32_t Nq,
                              int32_t Nkv, int32_t head_dim, float scale,
                              int64_t q_sb, int64_t q_sh, int64_t q_sn,
                              int64_t k_sb, int64_t k_sh, int64_t k_sn,
                              int64_t v_sb, int64_t v_sh, int64_t v_sn,
                              int64_t o_sb, int64_t o_sh, int64_t o_sn,
                              int32_t precision, void* stream);

/* 2D RoPE in place on t [B, N, ld], columns [0, H*64): per 64-wide head,
 * dims [0,32) rotate by the token's row y and [32,64) by its column x
 * (token n at (n / grid_w, n % grid_w)); within each 32-dim half, pairs
 * (j, j+16) rotate by pos * base^(-2j/32). Replaces the token-level CPU pass
 * MASt3REncoderV2#apply_rope (src/mastr/encoder_v2.cr:180-258). */
int32_t gs_hip_rope2d(float* t, int32_t B, int32_t N, int32_t H, int64_t ld,
                      int32_t grid_w, float base, void* stream);

/* NN::GPUOps.conv2d_forward (src/nn/gpu_ops.cr:478-527); the arithmetic of
 * Conv2DBlock#forward_cpu (src/mastr/decoder_v2.cr:281-344). x NHWC
 * [B,H,W,Cin], w OIHW [Cout,Cin,k,k] (w_layout 0) or OHWI [Cout,k,k,Cin]
 * (w_layout 1), y NHWC. Any Cin >= 1: the implicit-GEMM conv reads 32
 * channels per step from 16-byte aligned rows, so other channel counts (and
 * OIHW weights with k > 1, re-laid per call) run on zero-padded copies in
 * stream-ordered scratch. flags: GS_CONV_RELU_IN applies ReLU to x on load,
 * GS_CONV_RELU_OUT after the bias, residual (nullable) is added last. */
#define GS_CONV_RELU_IN 1
#define GS_CONV_RELU_OUT 2
#define GS_CONV_F32X6 4   /* products as GS_EPI_F32X6 */
int32_t gs_hip_conv2d(const float* x, int32_t B, int32_t H, int32_t W,
                      int32_t Cin, const float* w, const float* b, float* y,
                      int32_t Cout, int32_t k, int32_t stride, int32_t pad,
                      int32_t w_layout, int32_t flags, const float* residual,
                      void* stream);

/* gs_hip_conv2d with a kh x kw kernel: conv2d_forward reads kernel_h and
 * kernel_w from the weight's shape separately (src/nn/gpu_ops.cr:491-495),
 * with one stride and one padding for both axes. w OIHW [Cout,Cin,kh,kw]
 * (w_layout 0) or OHWI [Cout,kh,kw,Cin] (w_layout 1); output
 * Ho = (H + 2 pad - kh) / stride + 1, Wo = (W + 2 pad - kw) / stride + 1.
 * gs_hip_conv2d(..., k, ...) is gs_hip_conv2d_hw(..., k, k, ...). */
int32_t gs_hip_conv2d_hw(const float* x, int32_t B, int32_t H, int32_t W,
                         int32_t Cin, const float* w, const float* b, float* y,
                         int32_t Cout, int32_t kh, int32_t kw, int32_t stride,
                         int32_t pad, int32_t w_layout, int32_t flags,
                         const float* residual, void* stream);

/* ConvTranspose2d with kernel == stride (no padding), NHWC, weight in the
 * PyTorch layout [Cin, Cout, k, k]. Cin % 32 == 0, Cout % 32 == 0. */
int32_t gs_hip_conv_transpose(const float* x, int32_t B, int32_t H, int32_t W,
                              int32_t Cin, const float* w, const float* b,
                              float* y, int32_t Cout, int32_t k, void* stream);

/* Bilinear x2 upsample, align_corners=True, NHWC, C % 4 == 0. */
int32_t gs_hip_upsample2x(const float* x, int32_t B, int32_t H, int32_t W,
                          int32_t C, float* y, void* stream);

/* Caller-side passes of MASt3RInference, on the device (fp32, HBM-bound). */
/* resize_image (src/mastr/inference.cr:330-374) on F frames:
 * src [F, sh, sw, C] -> dst [F, th, tw, C]; bilinear with source coordinate
 * (t * (s-1)) / (t_n-1) in fp32, truncated and clamped to [0, s-2], and the
 * reference's four-term sum. sh, sw, th, tw >= 2. Bit-exact to the reference
 * arithmetic. */
int32_t gs_hip_resize_image(const float* src, int32_t F, int32_t sh,
                            int32_t sw, int32_t C, int32_t th, int32_t tw,
                            float* dst, void* stream);
/* preprocess_image (src/mastr/inference.cr:193-229): [B,H,W,3] in [0,1] ->
 * [B,3,H,W], (v - mean[c]) / std[c], ImageNet mean / std. */
int32_t gs_hip_preprocess_image(const float* src, int32_t B, int32_t H,
                                int32_t W, float* dst, void* stream);
/* resize_image then preprocess_image in one pass (the per-frame work of
 * frames_to_pointcloud, src/mastr/inference.cr:152-153 + 95-96):
 * [F, sh, sw, 3] -> [F, 3, th, tw]. Bit-identical to the two calls. */
int32_t gs_hip_prepare_frames(const float* src, int32_t F, int32_t sh,
                              int32_t sw, int32_t th, int32_t tw, float* dst,
                              void* stream);
/* collect_points (src/mastr/inference.cr:296-328) as an order-preserving
 * compaction: the points of pts [n,3] whose conf [n] is > threshold (strict;
 * NaN never selected) are appended, in element order, at out_pts[*count],
 * out_conf[*count]; *count (DEVICE int64, caller-zeroed before the first
 * call) advances by the selected number, also past capacity (positions >=
 * capacity are not written), so the caller can detect overflow. Its block
 * counts live in stream-ordered scratch (allocated and released on
 * `stream`), so calls on different streams are independent. */
int32_t gs_hip_collect_points(const float* pts, const float* conf, int64_t n,
                              float threshold, float* out_pts,
                              float* out_conf, int64_t capacity,
                              int64_t* count, void* stream);

/* gs_hip_collect_points without allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory at call time (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, behaviour and results as gs_hip_collect_points;
 * the block counts live in a static 256 KB device array of the library (one
 * per GPU, held until the process ends), so n is at most 2^27 (134217728)
 * points, and a larger n is an error before any launch. Calls share that
 * array per GPU: calls that overlap in time on one GPU (on different streams
 * or threads) race and must be ordered by the caller. */
#define GS_COLLECT_POINTS_NOALLOC_MAX ((int64_t)1 << 27)
int32_t gs_hip_collect_points_noalloc(const float* pts, const float* conf,
                                      int64_t n, float threshold,
                                      float* out_pts, float* out_conf,
                                      int64_t capacity, int64_t* count,
                                      void* stream);

/* ------------------------------------------------------------------------ */
/* 3. Graph-level entry points (MASt3R)                                      */
/* ------------------------------------------------------------------------ */

typedef struct gs_mastr_config {
  int32_t img_h, img_w, patch;
  int32_t enc_dim, enc_depth, enc_heads, enc_mlp;
  int32_t dec_dim, dec_depth, dec_heads, dec_mlp;
  int32_t dpt_feat;
  int32_t dpt_dims[4];
  int32_t dpt_hooks[4];
  int32_t head_mid;
  int32_t lf_hidden;
  int32_t desc_dim;
  float ln_eps;
  float rope_base;
  int32_t linear_layout; /* 0 = x W^T; 1 = reference CPU literal layout */
  int32_t rope_mode;     /* 0 none, 1 per-attention q/k 2D, 2 ref-token */
  int32_t precision;     /* 0 = fp32 MFMA; 1 = bf16-input / fp32-accumulate
                            MFMA GEMMs and attention (linear_layout 0 only);
                            2 = fp32 GEMMs and convolutions on bf16 matrix
                            cores through exact three-term bf16 splits of
                            both operands (six term products, fp32
                            accumulate; error vs fp64 at or below the fp32
                            MFMA kernels'), attention the same way
                            (fp32 MFMA for launches that split the keys)
                            (linear_layout 0 only) */
  int32_t composite;     /* 0 = MASt3R composition (full DPT at image
                            resolution, 1+exp confidence, descriptors, each
                            decoder chain attending to the other view's
                            previous state);
                            1 = the reference's literal forward_pair: each
                            chain attends to its own view's decoder_embed
                            output (src/mastr/decoder_v2.cr:170-191), stub DPT
                            at patch resolution (layer4_rn -> refinenet4 with
                            conv-ReLU-conv+x units -> ReLU, head.0, ReLU,
                            head.2, head.4), sigmoid confidence
                            (src/mastr/decoder_v2.cr:502-530, 619-655), no
                            descriptors. "ref512" = composite 1 at 512x512,
                            rope_mode 2, ln_eps 1e-5. */
} gs_mastr_config;

/* MASt3R ViT-L/ViT-B at 384x512 (24x32 patch grid), eps 1e-6, RoPE base 100,
 * DPT hooks {0,6,9,12}, fusion width 256, 24-channel descriptors. Mirrors
 * MASt3RInference#initialize (src/mastr/inference.cr:25-57). */
void gs_mastr_default_config(gs_mastr_config* cfg);

/* Weight inventory of a configuration, in checkpoint naming
 * (src/mastr/weight_loader.cr:43-123). kind: 0 weight ~ N(0, 0.02),
 * 1 bias (0), 2 LayerNorm gamma (1), 3 LayerNorm beta (0). shape has up to 4
 * dims, unused dims are 0. Returns -1 for i out of range. */
int32_t gs_mastr_weight_count(const gs_mastr_config* cfg);
int32_t gs_mastr_weight_info(const gs_mastr_config* cfg, int32_t i,
                             char* name_out, int32_t name_cap,
                             int64_t shape_out[4], int32_t* kind_out);
/* The host values of weight i for a seed: kind 0 -> N(0, 0.02); bias ->
 * N(0, bias_std) (0 when bias_std == 0); gamma -> 1 + N(0, ln_std); beta ->
 * N(0, ln_std). The configs' weights are seed 0, bias_std = ln_std = 0. */
int32_t gs_mastr_weight_values(const gs_mastr_config* cfg, int32_t i,
                               uint64_t seed, float bias_std, float ln_std,
                               float* host_out, int64_t n);

/* Context: device weights (re-laid for the kernels) + workspaces for up to
 * max_pairs pairs (including a 64 MB scratch for the split-K partial tiles
 * and key-range attention states of small launches). Weights start
 * uninitialised. A context's calls share its workspaces: calls on one
 * context must not overlap in time (one stream per context, or order them);
 * separate contexts are independent. */
int32_t gs_hip_mastr_create(const gs_mastr_config* cfg, int32_t max_pairs,
                            void** ctx_out);
void gs_hip_mastr_destroy(void* ctx);
/* Fill every weight from the seeded generator (see gs_mastr_weight_values). */
int32_t gs_hip_mastr_init_seeded(void* ctx, uint64_t seed, float bias_std,
                                 float ln_std);
/* Set one weight from host memory by checkpoint name (numel must match). */
int32_t gs_hip_mastr_set_weight(void* ctx, const char* name,
                                const float* host_values, int64_t numel);

/* MASt3REncoderBlockV2#forward (src/mastr/encoder_v2.cr:38-48), in place on
 * x [B, N, enc_dim] (device), block `layer` of the context. */
int32_t gs_hip_mastr_encoder_block(void* ctx, int32_t layer, float* x,
                                   int32_t B, void* stream);
/* MASt3REncoderV2#forward (src/mastr/encoder_v2.cr:135-148):
 * img [B,3,H,W] -> enc [B, N, enc_dim] (after enc_norm). B <= 2*max_pairs. */
int32_t gs_hip_mastr_encoder(void* ctx, const float* img, int32_t B,
                             float* enc, void* stream);
/* MASt3RInference#forward_pair (src/mastr/inference.cr:92-115) for B pairs:
 * img1, img2 [B,3,H,W] -> per view pts [B,H,W,3], conf [B,H,W,1] (1+exp),
 * desc [B,H,W,desc_dim]. Any output pointer may be NULL to skip that head.
 * composite 1: pts [B,gh,gw,3], conf [B,gh,gw,1] (sigmoid) on the patch grid
 * gh = H/patch, gw = W/patch; desc must be NULL. */
int32_t gs_hip_mastr_pair(void* ctx, const float* img1, const float* img2,
                          int32_t B, float* pts1, float* conf1, float* desc1,
                          float* pts2, float* conf2, float* desc2,
                          void* stream);
/* enable != 0: gs_hip_mastr_pair captures its launch sequence into a hipGraph
 * on the first call with a given (B, image / output pointers, stream) and
 * replays it while those repeat (re-capturing when they change). Needs a
 * non-null stream; calls made while gs_hip_profile_* is active run eagerly.
 * The weights may change between replays (the graph reads them in place). */
int32_t gs_hip_mastr_set_graph(void* ctx, int32_t enable);
/* Intermediate taps of the last gs_hip_mastr_pair call, copied to device
 * buffers: enc1/enc2 [B,N,enc_dim], dec1/dec2 = dec_norm output
 * [B,N,dec_dim]. Any pointer may be NULL. */
int32_t gs_hip_mastr_pair_taps(void* ctx, int32_t B, float* enc1, float* enc2,
                               float* dec1, float* dec2, void* stream);

/* MASt3RInference#frames_to_pointcloud (src/mastr/inference.cr:135-191):
 * F frames [F, src_h, src_w, 3] in [0,1] (device) are resized to the
 * context's image size and normalised once each; the F-1 consecutive pairs
 * run as batched pair calls of up to max_pairs pairs (no descriptor heads);
 * the view-1 points of every pair, then the view-2 points of the last pair,
 * with conf > threshold are compacted in order into out_pts [capacity, 3],
 * out_conf [capacity] (device). *n_points (host) receives the total count,
 * which may exceed capacity (then only the first capacity are written).
 * F < 2 gives 0 points. Synchronises the stream before returning; runs
 * eagerly even when graph replay is enabled. */
int32_t gs_hip_mastr_frames_to_pointcloud(void* ctx, const float* frames,
                                          int32_t F, int32_t src_h,
                                          int32_t src_w, float threshold,
                                          float* out_pts, float* out_conf,
                                          int64_t capacity, int64_t* n_points,
                                          void* stream);

/* Checkpoint ingestion. SafetensorsLoader (src/mastr/weights.cr:30-290):
 * u64-LE header length + JSON header {name: {dtype, shape, data_offsets}}
 * ("__metadata__" skipped) + raw data, mmapped; F32 / F16 / BF16 tensors read
 * as fp32 (F16 exactly, subnormals included; BF16 by a 16-bit shift). The
 * host-only calls need no GPU. A malformed file (offsets outside the data,
 * size not matching shape x dtype, bad JSON) is an error, not a partial read. */
int32_t gs_safetensors_count(const char* path);
/* Tensor i in header order: name (NUL-terminated, truncated to name_cap),
 * dtype string (up to 7 chars + NUL into dtype_out[8]), shape (up to 8 dims,
 * unused 0), ndim. */
int32_t gs_safetensors_info(const char* path, int32_t i, char* name_out,
                            int32_t name_cap, char* dtype_out,
                            int64_t shape_out[8], int32_t* ndim_out);
/* Tensor `name` converted to fp32 into host memory (numel must match). */
int32_t gs_safetensors_read_f32(const char* path, const char* name,
                                float* host_out, int64_t numel);
/* WeightLoader#load_* (src/mastr/weight_loader.cr:43-123): every tensor of the
 * file whose name is in the context's inventory is placed (its shape must
 * equal the inventory shape, else error); n_unexpected counts file tensors not in the inventory,
 * n_missing inventory weights absent from the file (left as they were). The
 * fused attn.qkv tensors are placed fused. Any count pointer may be NULL. */
int32_t gs_hip_mastr_load_safetensors(void* ctx, const char* path,
                                      int32_t* n_loaded, int32_t* n_unexpected,
                                      int32_t* n_missing);

/* ------------------------------------------------------------------------ */
/* 4. Measurement (no reference counterpart: the reference only wall-clocks  */
/*    whole ops, src/main.cr:860-909)                                         */
/* ------------------------------------------------------------------------ */
/* Between begin and end, every kernel launch is bracketed by HIP events on
 * its own stream. end synchronises those events and returns the number of
 * distinct kernels (per_shape != 0: distinct kernel + problem shape); entry i
 * gives its launches, summed event time (ms), summed algorithmic flops and
 * algorithmic HBM bytes. The profiler state is process-wide: one thread
 * brackets its own launches, and no other thread launches in between. */
int32_t gs_hip_profile_begin(int32_t per_shape);
int32_t gs_hip_profile_end(void);
int32_t gs_hip_profile_entry(int32_t i, char* name_out, int32_t name_cap,
                             int64_t* launches, double* ms, double* flops,
                             double* bytes);

#ifdef __cplusplus
}
#endif
#endif
