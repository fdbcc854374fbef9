// General-shape kernels of the op-level entry points: the shapes the tuned
// MFMA kernels do not take (any attention head_dim, any LayerNorm width,
// unaligned operands), and the staging copies that bring a ragged
// linear / convolution to the MFMA GEMM's operand contract (K a multiple of
// 32, 16-byte aligned rows).
//
// The reference's GPUOps accepts these shapes: fused_attention takes any
// head_dim (src/nn/gpu_ops.cr:200-227, the reference's own MHA spec runs
// head_dim 16, spec/nn/attention_spec.cr:49-58), linear_forward any in / out
// width (src/nn/gpu_ops.cr:39-78, linear_forward_simple below 64), and
// layernorm_forward any feature count (src/nn/gpu_ops.cr:114-138).
#include <math.h>

#include "internal.h"

namespace gs {
namespace {

constexpr int kGKT = 32;   // keys per LDS tile of the general attention
constexpr int kGHD = 128;  // head dims per LDS tile (and the register-accumulator form's limit)

// One wavefront per query, four queries per workgroup, K/V tiles of 32 keys
// staged through LDS for the four. Scores: lane t (and t + 32) of the wave
// holds key t of the tile, each half summing half the head dims, combined by
// one exchange. Online softmax with expf, then lane d accumulates output dims
// d and d + 64 over the tile's keys, the probabilities broadcast by shuffles.
__global__ __launch_bounds__(256) void attn_general_kernel(AttnArgs p, int32_t hd) {
  __shared__ float Ks[kGKT * (kGHD + 1)];
  __shared__ float Vs[kGKT * kGHD];
  __shared__ float Qs[4][kGHD];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int b = blockIdx.z, h = blockIdx.y;
  const int q = blockIdx.x * 4 + w;
  const bool qok = q < p.Nq;
  const float* qb = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const float* kb = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const float* vb = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  float* ob = p.o + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;
  if (qok)
    for (int d = lane; d < hd; d += 64) Qs[w][d] = qb[(int64_t)q * p.q_sn + d];
  const int ks = hd | 1;  // odd row stride: lanes reading one column of K hit distinct banks
  const int t = lane & 31, half = lane >> 5;
  const int d0 = half ? (hd >> 1) : 0, d1 = half ? hd : (hd >> 1);
  float m = -INFINITY, l = 0.f, o0 = 0.f, o1 = 0.f;
  for (int kbase = 0; kbase < p.Nkv; kbase += kGKT) {
    __syncthreads();  // previous tile consumed (and the Q rows written)
    for (int e = tid; e < kGKT * hd; e += 256) {
      const int kk = e / hd, d = e - kk * hd;
      const int key = kbase + kk;
      float kv = 0.f, vv = 0.f;
      if (key < p.Nkv) {
        kv = kb[(int64_t)key * p.k_sn + d];
        vv = vb[(int64_t)key * p.v_sn + d];
      }
      Ks[kk * ks + d] = kv;
      Vs[kk * hd + d] = vv;
    }
    __syncthreads();
    if (!qok) continue;  // wave-uniform; the barriers above are reached by every wave
    const int key = kbase + t;
    float sc = 0.f;
    for (int d = d0; d < d1; ++d) sc += Qs[w][d] * Ks[t * ks + d];
    sc += __shfl_xor(sc, 32);
    sc = key < p.Nkv ? sc * p.scale : -INFINITY;
    float mb = sc;
    for (int off = 16; off > 0; off >>= 1) mb = fmaxf(mb, __shfl_xor(mb, off));
    const float mn = fmaxf(m, mb);  // finite: every tile holds at least one key
    const float alpha = expf(m - mn);
    const float pt = expf(sc - mn);
    float ps = pt;
    for (int off = 16; off > 0; off >>= 1) ps += __shfl_xor(ps, off);
    l = l * alpha + ps;
    o0 *= alpha;
    o1 *= alpha;
    for (int j = 0; j < kGKT; ++j) {
      const float pj = __shfl(pt, j);
      if (lane < hd) o0 += pj * Vs[j * hd + lane];
      if (lane + 64 < hd) o1 += pj * Vs[j * hd + lane + 64];
    }
    m = mn;
  }
  if (!qok) return;
  float* orow = ob + (int64_t)q * p.o_sn;
  if (lane < hd) orow[lane] = o0 / l;
  if (lane + 64 < hd) orow[lane + 64] = o1 / l;
}

// head_dim > 128: the same tiling with the head dims taken in chunks of 128.
// Per tile of 32 keys, the scores accumulate over the chunks of Q and K
// (each chunk staged through LDS, the two half-waves splitting it as above);
// then, chunk by chunk of V, each lane rescales and accumulates output dims
// c0 + lane and c0 + lane + 64 in the query's own output row, which serves as
// the accumulator (only that lane reads and writes those addresses, so program
// order keeps them consistent); a last pass divides the row by the softmax
// sum. No head_dim limit beyond the 32-bit index range.
__global__ __launch_bounds__(256) void attn_general_wide_kernel(AttnArgs p, int32_t hd) {
  __shared__ float Ks[kGKT * (kGHD + 1)];
  __shared__ float Vs[kGKT * kGHD];
  __shared__ float Qs[4][kGHD];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int b = blockIdx.z, h = blockIdx.y;
  const int q = blockIdx.x * 4 + w;
  const bool qok = q < p.Nq;
  const float* qb = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const float* kb = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const float* vb = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  float* orow = p.o + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh + (int64_t)(qok ? q : 0) * p.o_sn;
  const int t = lane & 31, half = lane >> 5;
  float m = -INFINITY, l = 0.f;
  for (int kbase = 0; kbase < p.Nkv; kbase += kGKT) {
    const int key = kbase + t;
    float sc = 0.f;
    for (int c0 = 0; c0 < hd; c0 += kGHD) {
      const int cw = min(kGHD, hd - c0), ks = cw | 1;
      __syncthreads();  // previous chunk consumed
      for (int e = tid; e < kGKT * cw; e += 256) {
        const int kk = e / cw, d = e - kk * cw;
        const int kkey = kbase + kk;
        Ks[kk * ks + d] = kkey < p.Nkv ? kb[(int64_t)kkey * p.k_sn + c0 + d] : 0.f;
      }
      if (qok)
        for (int d = lane; d < cw; d += 64) Qs[w][d] = qb[(int64_t)q * p.q_sn + c0 + d];
      __syncthreads();
      const int d0 = half ? (cw >> 1) : 0, d1 = half ? cw : (cw >> 1);
      if (qok)
        for (int d = d0; d < d1; ++d) sc += Qs[w][d] * Ks[t * ks + d];
    }
    sc += __shfl_xor(sc, 32);
    sc = key < p.Nkv ? sc * p.scale : -INFINITY;
    float mb = sc;
    for (int off = 16; off > 0; off >>= 1) mb = fmaxf(mb, __shfl_xor(mb, off));
    const float mn = fmaxf(m, mb);  // finite: every tile holds at least one key
    const float alpha = expf(m - mn);
    const float pt = expf(sc - mn);
    float ps = pt;
    for (int off = 16; off > 0; off >>= 1) ps += __shfl_xor(ps, off);
    l = l * alpha + ps;
    for (int c0 = 0; c0 < hd; c0 += kGHD) {
      const int cw = min(kGHD, hd - c0);
      __syncthreads();  // K / previous V chunk consumed
      for (int e = tid; e < kGKT * cw; e += 256) {
        const int kk = e / cw, d = e - kk * cw;
        const int kkey = kbase + kk;
        Vs[kk * cw + d] = kkey < p.Nkv ? vb[(int64_t)kkey * p.v_sn + c0 + d] : 0.f;
      }
      __syncthreads();
      if (!qok) continue;  // wave-uniform; every wave reaches the barriers above
      // the first tile starts the accumulators at zero (the row holds no state yet)
      float o0 = 0.f, o1 = 0.f;
      if (kbase > 0) {
        if (lane < cw) o0 = orow[c0 + lane] * alpha;
        if (lane + 64 < cw) o1 = orow[c0 + lane + 64] * alpha;
      }
      for (int j = 0; j < kGKT; ++j) {
        const float pj = __shfl(pt, j);
        if (lane < cw) o0 += pj * Vs[j * cw + lane];
        if (lane + 64 < cw) o1 += pj * Vs[j * cw + lane + 64];
      }
      if (lane < cw) orow[c0 + lane] = o0;
      if (lane + 64 < cw) orow[c0 + lane + 64] = o1;
    }
    m = mn;
  }
  if (!qok) return;
  for (int d = lane; d < hd; d += 64) orow[d] = orow[d] / l;
}

__device__ __forceinline__ float block_sum_256(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();  // red is reused by the next reduction
  return t;
}

// One workgroup per row, any width D and alignment: two-pass mean / variance
// (LayerNorm#forward_cpu, src/nn/layernorm.cr:192-240), scalar loads.
__global__ __launch_bounds__(256) void layernorm_rows_kernel(LnArgs p) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int D = p.D;
  const float* x = p.x + row * D;
  float s = 0.f;
  for (int i = threadIdx.x; i < D; i += 256) s += x[i];
  const float mean = block_sum_256(s, red) / (float)D;
  float q = 0.f;
  for (int i = threadIdx.x; i < D; i += 256) {
    const float a = x[i] - mean;
    q += a * a;
  }
  const float var = block_sum_256(q, red) / (float)D;
  const float inv = 1.0f / sqrtf(var + p.eps);
  if (p.stats && threadIdx.x == 0) {
    p.stats[2 * row] = mean;
    p.stats[2 * row + 1] = inv;
  }
  if (!p.y) return;
  float* y = p.y + row * D;
  for (int i = threadIdx.x; i < D; i += 256) y[i] = (x[i] - mean) * inv * p.gamma[i] + p.beta[i];
}

// dst[r, c] (row length cp) = src[r * s_row + c * s_col] for c < cols, 0 for
// cols <= c < cp: a zero-padded, possibly transposing copy into a dense
// 16-byte aligned operand.
__global__ void stage_kernel(const float* __restrict__ src, int64_t rows, int64_t cols,
                             int64_t s_row, int64_t s_col, float* __restrict__ dst, int64_t cp) {
  const int64_t total = rows * cp;
  for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = id / cp, c = id - r * cp;
    dst[id] = c < cols ? src[r * s_row + c * s_col] : 0.f;
  }
}

// Convolution weight OIHW (layout 0) or OHWI (layout 1) [Cout, ...] of
// KH x KW taps -> OHWI with the input channels zero-padded to cp:
// out[((oc*KH + kh)*KW + kw)*cp + ic].
__global__ void conv_weight_stage_kernel(const float* __restrict__ w, int32_t Cout, int32_t Cin,
                                         int32_t KH, int32_t KW, int32_t layout, int32_t cp,
                                         float* __restrict__ out) {
  const int64_t total = (int64_t)Cout * KH * KW * cp;
  for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (int64_t)gridDim.x * blockDim.x) {
    const int ic = (int)(id % cp);
    int64_t r = id / cp;
    const int kw = (int)(r % KW);
    r /= KW;
    const int kh = (int)(r % KH);
    const int64_t oc = r / KH;
    float v = 0.f;
    if (ic < Cin)
      v = layout == 0 ? w[((oc * Cin + ic) * KH + kh) * KW + kw]
                      : w[((oc * KH + kh) * KW + kw) * Cin + ic];
    out[id] = v;
  }
}

unsigned stride_grid(int64_t total) {
  const int64_t b = (total + 255) / 256;
  return (unsigned)(b < 16384 ? (b > 0 ? b : 1) : 16384);
}

}  // namespace

int launch_attention_general(const AttnArgs& a, int32_t hd, hipStream_t s) {
  GS_REQUIRE(hd >= 1, "attention: head_dim must be >= 1");
  GS_REQUIRE(a.q && a.k && a.v && a.o, "attention: null operand");
  GS_REQUIRE(a.B > 0 && a.H > 0 && a.Nq > 0 && a.Nkv > 0, "attention: bad sizes");
  GS_REQUIRE(a.B <= 65535 && a.H <= 65535, "attention: grid too large");
  const int64_t st[12] = {a.q_sb, a.q_sh, a.q_sn, a.k_sb, a.k_sh, a.k_sn,
                          a.v_sb, a.v_sh, a.v_sn, a.o_sb, a.o_sh, a.o_sn};
  for (int j = 0; j < 12; ++j) GS_REQUIRE(st[j] >= 0, "attention: negative stride");
  dim3 grid((unsigned)((a.Nq + 3) / 4), a.H, a.B), block(256);
  hipEvent_t ev = prof_start(s);
  if (hd <= kGHD)
    hipLaunchKernelGGL(attn_general_kernel, grid, block, 0, s, a, hd);
  else
    hipLaunchKernelGGL(attn_general_wide_kernel, grid, block, 0, s, a, hd);
  GS_CHECK_HIP(hipGetLastError());
  const double units = (double)a.B * a.H;
  prof_stop(s, ev, hd <= kGHD ? "attn_general_kernel" : "attn_general_wide_kernel",
            units * 4.0 * a.Nq * (double)a.Nkv * hd, units * hd * (8.0 * a.Nq + 8.0 * a.Nkv));
  return 0;
}

int launch_layernorm_rows(const LnArgs& a, hipStream_t s) {
  GS_REQUIRE(a.x && (a.y || a.stats) && a.gamma && a.beta, "layernorm: null operand");
  GS_REQUIRE(a.D > 0 && a.rows >= 0 && a.rows < INT32_MAX, "layernorm: bad sizes");
  GS_REQUIRE(!a.y_bf16, "layernorm: bf16 output needs D % 4 == 0 and aligned rows");
  if (a.rows == 0) return 0;
  hipEvent_t ev = prof_start(s);
  hipLaunchKernelGGL(layernorm_rows_kernel, dim3((unsigned)a.rows), dim3(256), 0, s, a);
  GS_CHECK_HIP(hipGetLastError());
  prof_stop(s, ev, "layernorm_rows_kernel", 8.0 * (double)a.rows * a.D,
            12.0 * (double)a.rows * a.D + 8.0 * a.D);
  return 0;
}

int launch_stage(const float* src, int64_t rows, int64_t cols, int64_t s_row, int64_t s_col,
                 float* dst, int64_t cp, hipStream_t s) {
  GS_REQUIRE(rows >= 0 && cols >= 0 && cp >= cols && src && dst, "stage: bad arguments");
  if (rows * cp == 0) return 0;
  hipLaunchKernelGGL(stage_kernel, dim3(stride_grid(rows * cp)), dim3(256), 0, s, src, rows, cols,
                     s_row, s_col, dst, cp);
  GS_CHECK_HIP(hipGetLastError());
  return 0;
}

int launch_conv_weight_stage(const float* w, int32_t Cout, int32_t Cin, int32_t kh, int32_t kw,
                             int32_t layout, int32_t cp, float* out, hipStream_t s) {
  GS_REQUIRE(w && out && Cout > 0 && Cin > 0 && kh > 0 && kw > 0 && cp >= Cin,
             "conv weight: bad arguments");
  const int64_t total = (int64_t)Cout * kh * kw * cp;
  hipLaunchKernelGGL(conv_weight_stage_kernel, dim3(stride_grid(total)), dim3(256), 0, s, w, Cout,
                     Cin, kh, kw, layout, cp, out);
  GS_CHECK_HIP(hipGetLastError());
  return 0;
}

}  // namespace gs
