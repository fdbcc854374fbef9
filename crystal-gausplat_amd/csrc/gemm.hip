// fp32 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x2_f32), LDS-staged.
//
// Covers every Linear of the path (NN::Linear#forward, src/nn/linear.cr:41-63,
// whose GPU seam is GPUOps.linear_forward, src/nn/gpu_ops.cr:39-78) and every
// DPT convolution as an implicit GEMM (Conv2DBlock#forward,
// src/mastr/decoder_v2.cr:241-344; GPUOps.conv2d_forward,
// src/nn/gpu_ops.cr:478-527), with the reference's CPU-side passes (bias,
// GELU, ReLU, residual add, RoPE) fused into the epilogue.
//
// Tiling: 256 threads = 4 wavefronts in a 2x2 arrangement, workgroup tile
// 128x128, K step 32. Each wavefront owns a 64x64 sub-tile = 2x2 MFMA 32x32
// blocks (64 accumulator registers per lane). Within one K step of 32, lane l
// (half h = l/32) feeds MFMA step t (0..15) with k = 16h + t, so every lane
// reads 16 contiguous k of its row: four ds_read_b128 per operand per step.
// LDS rows are padded to 36 floats so the 8 lanes of each ds_read_b128 phase
// hit 32 distinct banks. The next K step is prefetched into registers while
// the current one runs on the matrix cores.
#include <algorithm>
#include <string>

#include "bf16_split.h"
#include "internal.h"

typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace gs {
namespace {

constexpr int BM = 128, BN = 128, BK = 32, LDS = BK + 4;
constexpr int GROUP_M = 8;

// GELU, tanh form (src/nn/vit.cr:130-148): 0.5*v*(1 + tanh(u)) with
// u = c*(v + 0.044715*v^3), c = (float)sqrt(2/pi). Evaluated through the exact
// identity 0.5*(1 + tanh(u)) = 1/(1 + exp(-2u)) with the hardware exp2 and
// reciprocal (a few instructions instead of a library tanh in every epilogue
// element); the relative error is a few ulp, far inside the fp32 parity
// tolerance. Saturates to v for large u and to -0 for large negative u.
__device__ __forceinline__ float gelu_tanh(float v) {
  const float c = 0.7978845608028654f;
  const float u = c * (v + 0.044715f * v * v * v);
  const float e = __builtin_amdgcn_exp2f(-2.8853900817779268f * u);  // exp(-2u)
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}

// q = n / d, r = n % d for 0 <= n < 2^22, d >= 1, from rd = 1/d in fp32: the
// product n*rd is within 0.5 of n/d in that range, so one correction step
// makes the quotient exact.
__device__ __forceinline__ int divmod_small(int n, int d, float rd, int& r) {
  int q = (int)((float)n * rd);
  r = n - q * d;
  if (r < 0) {
    --q;
    r += d;
  } else if (r >= d) {
    ++q;
    r -= d;
  }
  return q;
}

__device__ __forceinline__ fx4 relu4(fx4 v) {
  return mk4(fmaxf(v.x, 0.f), fmaxf(v.y, 0.f), fmaxf(v.z, 0.f),
                     fmaxf(v.w, 0.f));
}

// Bias, RoPE, GELU / ReLU, residuals and the (scatter) store of a wave's
// 64x64 sub-tile. Accumulator layout of a 32x32 block: lane l, register r
// holds row 8*(r/4) + 4*(l/32) + (r%4), column l%32.
// Every operand a block needs (bias, RoPE table entries, residuals) is read
// into registers before its first store: the residual may alias C, so a load
// placed after a store could not be moved above it, and the 16 rows of a
// block would pay 16 serial memory latencies. Each element of C depends only
// on the same element of the residuals, so reading them all first is exact
// also in place. Addresses are clamped into the operands; out-of-range rows
// and columns are not stored.
// ROPE selects the RoPE form (no residuals, checked on the host); the two
// forms are separate branches so that their registers are not live together.
template <bool ROPE>
__device__ __forceinline__ void gemm_epilogue_t(const GemmArgs& p, const floatx16& acc00,
                                                const floatx16& acc01, const floatx16& acc10,
                                                const floatx16& acc11, int m0, int n0, int wm,
                                                int wn, int l32, int hl) {
  const int M = p.M, N = p.N;
  const int flags = ROPE ? p.flags & ~(EPI_RES1 | EPI_RES2) : p.flags & ~EPI_ROPE;
  float bval[2];
#pragma unroll
  for (int bj = 0; bj < 2; ++bj) {
    const int col = n0 + wn * 64 + bj * 32 + l32;
    bval[bj] = (flags & EPI_BIAS) ? p.bias[min(col, N - 1)] : 0.f;
  }
  // RoPE positions: when the tokens per image and the grid width are
  // multiples of 4, the 4 consecutive rows of a lane's row group (first row a
  // multiple of 4) lie in one image and one grid row at consecutive columns,
  // so the row -> (y, x) decode runs once per group
  const bool rope_fast = ROPE && (p.tok_per_img & 3) == 0 && (p.grid_w & 3) == 0;
  const float rtok = ROPE ? 1.0f / (float)p.tok_per_img : 0.f;
  const float rgw = ROPE ? 1.0f / (float)p.grid_w : 0.f;
#pragma unroll
  for (int bi = 0; bi < 2; ++bi) {
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
      const floatx16 c = bi == 0 ? (bj == 0 ? acc00 : acc01) : (bj == 0 ? acc10 : acc11);
      const int cblk = n0 + wn * 64 + bj * 32;
      const int col = cblk + l32;
      const int colc = min(col, N - 1);
      const int row0 = m0 + wm * 64 + bi * 32 + 4 * hl;
      const bool rope = ROPE && cblk < p.rope_ncols;
      // scatter column decode (wave-uniform kind, per-lane values)
      int sc_i = 0, sc_j = 0, sc_c = 0;
      if (flags & EPI_SCATTER) {
        const int s = col / p.sc_C;
        sc_c = col - s * p.sc_C;
        sc_i = s / p.sc_r;
        sc_j = s - sc_i * p.sc_r;
      }
      // Half a block (8 rows) at a time: its residuals are read into
      // registers first (x: residual 1, y: residual 2), and the RoPE table
      // entries of its rows (cos / sin at the row's position on the block's
      // axis, frequency l32 % 16).
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float x[8], y[8];
        float rcs[8], rsn[8];
        if (rope) {
          const int f = l32 & 15;
          const bool xaxis = (cblk >> 5) & 1;
          if (rope_fast) {
#pragma unroll
            for (int gg = 0; gg < 2; ++gg) {
              int tok, tx;
              divmod_small(row0 + 8 * (2 * h + gg), p.tok_per_img, rtok, tok);
              const int ty = divmod_small(tok, p.grid_w, rgw, tx);
              if (xaxis) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  rcs[4 * gg + e] = p.rope_cos[(tx + e) * 16 + f];
                  rsn[4 * gg + e] = p.rope_sin[(tx + e) * 16 + f];
                }
              } else {
                const float cs = p.rope_cos[ty * 16 + f], sn = p.rope_sin[ty * 16 + f];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  rcs[4 * gg + e] = cs;
                  rsn[4 * gg + e] = sn;
                }
              }
            }
          } else {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              const int r = 8 * h + u;
              int tok, tx;
              divmod_small(row0 + 8 * (r >> 2) + (r & 3), p.tok_per_img, rtok, tok);
              const int ty = divmod_small(tok, p.grid_w, rgw, tx);
              const int pos = xaxis ? tx : ty;
              rcs[u] = p.rope_cos[pos * 16 + f];
              rsn[u] = p.rope_sin[pos * 16 + f];
            }
          }
        }
        if (flags & EPI_RES1) {
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int r = 8 * h + u;
            const int row = min(row0 + 8 * (r >> 2) + (r & 3), M - 1);
            x[u] = p.R1[(int64_t)row * p.ldr1 + colc];
          }
        }
        if (flags & EPI_RES2) {
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int r = 8 * h + u;
            const int row = min(row0 + 8 * (r >> 2) + (r & 3), M - 1);
            y[u] = p.R2[(int64_t)row * p.ldr2 + colc];
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int r = 8 * h + u;
          const int row = row0 + 8 * (r >> 2) + (r & 3);
          float v = c[r];
          if (flags & EPI_BIAS) v = v + bval[bj];
          if (rope) {
            const float partner = __shfl_xor(v, 16);
            v = (l32 < 16) ? (v * rcs[u] - partner * rsn[u]) : (v * rcs[u] + partner * rsn[u]);
          }
          if (flags & EPI_GELU) v = gelu_tanh(v);
          if (flags & EPI_RELU) v = fmaxf(v, 0.f);
          if (row < M && col < N) {
            if (flags & EPI_RES1) v = v + x[u];
            if (flags & EPI_RES2) v = y[u] + v;
            if (flags & EPI_SCATTER) {
              if (sc_c < p.sc_Cout) {
                const int hw = p.sc_gh * p.sc_gw;
                const int img = row / hw;
                const int rem = row - img * hw;
                const int yy = rem / p.sc_gw, xx = rem - (rem / p.sc_gw) * p.sc_gw;
                const int64_t oy = (int64_t)img * p.sc_gh * p.sc_r + yy * p.sc_r + sc_i;
                const int64_t ox = (int64_t)xx * p.sc_r + sc_j;
                const int64_t si = (oy * p.sc_gw * p.sc_r + ox) * p.sc_Cout + sc_c;
                if (flags & EPI_BF16OUT)
                  ((__bf16*)p.C)[si] = (__bf16)v;
                else
                  p.C[si] = v;
              }
            } else if (flags & EPI_BF16OUT) {
              ((__bf16*)p.C)[(int64_t)row * p.ldc + col] = (__bf16)v;
            } else {
              p.C[(int64_t)row * p.ldc + col] = v;
              if (flags & EPI_DUAL) {
                if (flags & EPI_DUAL_RELU_H)
                  ((__bf16*)p.C2)[(int64_t)row * p.ldc + col] = (__bf16)fmaxf(v, 0.f);
                else
                  p.C2[(int64_t)row * p.ldc + col] = v;
              }
            }
          }
        }
      }
    }
  }
}

__device__ __forceinline__ void gemm_epilogue(const GemmArgs& p, const floatx16& acc00,
                                              const floatx16& acc01, const floatx16& acc10,
                                              const floatx16& acc11, int m0, int n0, int wm,
                                              int wn, int l32, int hl) {
  if (p.flags & EPI_ROPE)
    gemm_epilogue_t<true>(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
  else
    gemm_epilogue_t<false>(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
}

// EPI_DUAL's second store of four consecutive columns at element offset off:
// the value, or with EPI_DUAL_RELU_H bf16(max(v, 0)) (C2 then holds bf16).
__device__ __forceinline__ void dual_store(const GemmArgs& p, int flags, int64_t off, fx4 v) {
  if (flags & EPI_DUAL_RELU_H) {
    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
    const fx4 r = relu4(v);
    const bf16x4_t h = {(__bf16)r.x, (__bf16)r.y, (__bf16)r.z, (__bf16)r.w};
    *(bf16x4_t*)((__bf16*)p.C2 + off) = h;
  } else {
    *(fx4*)(p.C2 + off) = v;
  }
}

// Split-K range of workgroup row blockIdx.y: the K steps (of `unit` elements)
// are cut at floor(y * steps / S), so ranges differ by at most one step and S
// need not divide the step count (the host keeps every range non-empty).
__device__ __forceinline__ void split_range(int K, int S, int unit, int& kbeg, int& kend) {
  const int steps = K / unit, y = blockIdx.y;
  kbeg = (int)((int64_t)y * steps / S) * unit;
  kend = (int)((int64_t)(y + 1) * steps / S) * unit;
}

// Split-K: the raw accumulators of K range blockIdx.y go to
// part[blockIdx.y][row][col]; gemm_splitk_reduce applies the epilogue.
__device__ __forceinline__ void store_partial(const GemmArgs& p, const floatx16& acc00,
                                              const floatx16& acc01, const floatx16& acc10,
                                              const floatx16& acc11, int m0, int n0, int wm,
                                              int wn, int l32, int hl) {
  float* part = p.part + (int64_t)blockIdx.y * p.M * p.N;
#pragma unroll
  for (int bi = 0; bi < 2; ++bi) {
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
      const floatx16 c = bi == 0 ? (bj == 0 ? acc00 : acc01) : (bj == 0 ? acc10 : acc11);
      const int col = n0 + wn * 64 + bj * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + bi * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
        if (row < p.M && col < p.N) part[(int64_t)row * p.N + col] = c[r];
      }
    }
  }
}

// Sum of the ksplit partials in split order, then the epilogue of
// gemm_epilogue in the same operation order (bias, RoPE, GELU / ReLU,
// residuals, store, dual store). One thread per 4 consecutive columns; RoPE
// reads the partner columns (col ^ 16) the same way. N % 4 == 0, no scatter.
// The loads go out four (then two) at a time before their adds (a load-add
// loop waits for each partial in turn); the adds keep the split order.
__device__ __forceinline__ fx4 splitk_sum(const GemmArgs& p, int S, int64_t off) {
  const int64_t plane = (int64_t)p.M * p.N;
  const float* q = p.part + off;
  fx4 v = *(const fx4*)q;
  int s = 1;
  for (; s + 3 < S; s += 4) {
    const fx4 a = *(const fx4*)(q + s * plane), b = *(const fx4*)(q + (s + 1) * plane);
    const fx4 c = *(const fx4*)(q + (s + 2) * plane), d = *(const fx4*)(q + (s + 3) * plane);
    v = v + a;
    v = v + b;
    v = v + c;
    v = v + d;
  }
  if (s + 1 < S) {
    const fx4 a = *(const fx4*)(q + s * plane), b = *(const fx4*)(q + (s + 1) * plane);
    v = v + a;
    v = v + b;
    s += 2;
  }
  if (s < S) v = v + *(const fx4*)(q + s * plane);
  return v;
}

__global__ __launch_bounds__(256) void gemm_splitk_reduce(GemmBatch batch) {
  const GemmArgs& p = batch.g[blockIdx.z];
  const int nq = p.N >> 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.M * nq) return;
  const int row = (int)(i / nq), c0 = (int)(i - (int64_t)row * nq) * 4;
  const int S = batch.ksplit, flags = p.flags;
  fx4 v = splitk_sum(p, S, (int64_t)row * p.N + c0);
  if (flags & EPI_BIAS) v = v + *(const fx4*)(p.bias + c0);
  const int cblk = c0 & ~31;
  if ((flags & EPI_ROPE) && cblk < p.rope_ncols) {
    const int cp = c0 ^ 16;
    fx4 w = splitk_sum(p, S, (int64_t)row * p.N + cp);
    if (flags & EPI_BIAS) w = w + *(const fx4*)(p.bias + cp);
    const int tok = row % p.tok_per_img;
    const int ty = tok / p.grid_w, tx = tok - ty * p.grid_w;
    const int pos = ((cblk >> 5) & 1) ? tx : ty;
    const bool first = (c0 & 31) < 16;
    float out[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int f = (c0 + u) & 15;
      const float cs = p.rope_cos[pos * 16 + f], sn = p.rope_sin[pos * 16 + f];
      out[u] = first ? (v[u] * cs - w[u] * sn) : (v[u] * cs + w[u] * sn);
    }
    v = mk4(out[0], out[1], out[2], out[3]);
  }
  if (flags & EPI_GELU) v = mk4(gelu_tanh(v.x), gelu_tanh(v.y), gelu_tanh(v.z), gelu_tanh(v.w));
  if (flags & EPI_RELU) v = relu4(v);
  if (flags & EPI_RES1) v = v + *(const fx4*)(p.R1 + (int64_t)row * p.ldr1 + c0);
  if (flags & EPI_RES2) v = *(const fx4*)(p.R2 + (int64_t)row * p.ldr2 + c0) + v;
  if (flags & EPI_BF16OUT) {
    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
    bf16x4_t h;
    h.x = (__bf16)v.x;
    h.y = (__bf16)v.y;
    h.z = (__bf16)v.z;
    h.w = (__bf16)v.w;
    *(bf16x4_t*)((__bf16*)p.C + (int64_t)row * p.ldc + c0) = h;
    return;
  }
  *(fx4*)(p.C + (int64_t)row * p.ldc + c0) = v;
  if (flags & EPI_DUAL) dual_store(p, flags, (int64_t)row * p.ldc + c0, v);
}

// gemm_splitk_reduce for launches with EPI_LNOUT: one wavefront per output row
// (columns 4 * (lane + 64 i)) sums the partials in split order and applies
// the bias / residual epilogue in gemm_splitk_reduce's order, stores the row,
// then writes its LayerNorm with layernorm_kernel's per-lane sums, wavefront
// reduction and expression, so both outputs are bit-identical to the reduce
// pass followed by the LayerNorm kernel. N <= 256 * NV, N % 4 == 0.
template <int NV>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_ln(GemmBatch batch) {
  const GemmArgs& p = batch.g[blockIdx.y];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= p.M) return;
  const int N = p.N, nv = N >> 2, S = batch.ksplit, flags = p.flags;
  fx4 v[NV];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    if (idx < nv) {
      const int c0 = 4 * idx;
      fx4 x = splitk_sum(p, S, row * N + c0);
      if (flags & EPI_BIAS) x = x + *(const fx4*)(p.bias + c0);
      if (flags & EPI_RES1) x = x + *(const fx4*)(p.R1 + row * p.ldr1 + c0);
      if (flags & EPI_RES2) x = *(const fx4*)(p.R2 + row * p.ldr2 + c0) + x;
      *(fx4*)(p.C + row * p.ldc + c0) = x;
      v[i] = x;
      s += x.x + x.y + x.z + x.w;
    } else {
      v[i] = mk4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const float mean = wave_sum(s) / (float)N;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    if (idx < nv) {
      const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
      q += a * a + b * b + c * c + d * d;
    }
  }
  const float var = wave_sum(q) / (float)N;
  const float inv = 1.0f / sqrtf(var + p.lnout_eps);
  const fx4* g4 = (const fx4*)p.lnout_g;
  const fx4* b4 = (const fx4*)p.lnout_b;
  fx4* yr = (fx4*)(p.lnout + row * N);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    if (idx < nv) {
      const fx4 g = g4[idx], bb = b4[idx];
      fx4 o;
      o.x = (v[i].x - mean) * inv * g.x + bb.x;
      o.y = (v[i].y - mean) * inv * g.y + bb.y;
      o.z = (v[i].z - mean) * inv * g.z + bb.z;
      o.w = (v[i].w - mean) * inv * g.w + bb.w;
      yr[idx] = o;
    }
  }
}

// Global loads of one K step into registers (macros rather than lambdas so the
// register arrays stay in VGPRs). They use the kernel's per-row state
// (arow, aval, ohs/ows/cbase, lnm/lnr, boff, bncol). GS_LOAD_A only issues the
// loads (raw values into ra, the LayerNorm affine columns into lgb, the conv
// tap validity into aok); GS_FIX_A applies the LayerNorm, the padding zeros
// and the ReLU prologue when the step is written to LDS, so no arithmetic
// waits on a prefetch at the point where it is issued.
#define GS_LOAD_A(K0)                                                                    \
  {                                                                                      \
    const int k0_ = (K0);                                                                \
    if (ALOAD == A_LN) {                                                                 \
      lgb[0] = *(const fx4*)(p.ln_g + k0_ + lc4);                                        \
      lgb[1] = *(const fx4*)(p.ln_b + k0_ + lc4);                                        \
    }                                                                                    \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                      \
      if (ALOAD == A_PLAIN || ALOAD == A_LN) {                                           \
        ra[i] = *(const fx4*)(p.A + (int64_t)arow[i] * p.lda + k0_ + lc4);               \
      } else if (ALOAD == A_CONCAT) {                                                    \
        const bool first = k0_ < p.K1;                                                   \
        const float* base = first ? p.A : p.A2;                                          \
        const int64_t ld = first ? p.lda : p.lda2;                                       \
        const int kc = first ? k0_ : k0_ - p.K1;                                         \
        ra[i] = *(const fx4*)(base + (int64_t)arow[i] * ld + kc + lc4);                  \
      } else {                                                                           \
        /* tap (kh, kw), channels ic0..: one offset on the row's base; */                \
        /* padded taps read A[lc4..] (in bounds) and are zeroed by GS_FIX_A */           \
        const int kk = k0_ / p.cCin;                                                     \
        const int ic0 = k0_ - kk * p.cCin;                                               \
        const int kh = kk / p.ckw, kw = kk - kh * p.ckw;                                   \
        const int64_t toff = ((int64_t)kh * p.cW + kw) * p.cCin + ic0;                   \
        const int ih = ohs[i] + kh, iw = ows[i] + kw;                                    \
        const bool ok = aval[i] && (unsigned)ih < (unsigned)p.cH && (unsigned)iw < (unsigned)p.cW; \
        aok[i] = ok;                                                                     \
        ra[i] = *(const fx4*)(p.A + (ok ? cbase[i] + toff : 0) + lc4);                   \
      }                                                                                  \
    }                                                                                    \
  }
#define GS_FIX_A()                                                                       \
  _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                        \
    fx4 v = ra[i];                                                                       \
    if (ALOAD == A_LN) {                                                                 \
      const fx4 g_ = lgb[0], b_ = lgb[1];                                                \
      v.x = (v.x - lnm[i]) * lnr[i] * g_.x + b_.x;                                       \
      v.y = (v.y - lnm[i]) * lnr[i] * g_.y + b_.y;                                       \
      v.z = (v.z - lnm[i]) * lnr[i] * g_.z + b_.z;                                       \
      v.w = (v.w - lnm[i]) * lnr[i] * g_.w + b_.w;                                       \
    }                                                                                    \
    if (ALOAD == A_CONV) v = aok[i] ? v : zero4; /* padded tap */                        \
    if (A_RELU) v = relu4(v);                                                            \
    ra[i] = v;                                                                           \
  }

#define GS_LOAD_B_F32(K0)                                                                \
  {                                                                                      \
    const int k0_ = (K0);                                                                \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                      \
      if (BLAYOUT == B_NT) {                                                             \
        const fx4 w = *(const fx4*)(p.B + boff[i] + k0_);                                \
        rb[i] = w;                                                                       \
      } else {                                                                           \
        const int kb = (tid >> 5) + 8 * i;                                               \
        const fx4 w = *(const fx4*)(p.B + (int64_t)(k0_ + kb) * p.ldb + bncol);          \
        rb[i] = w;                                                                       \
      }                                                                                  \
    }                                                                                    \
  }

// Per-row load state shared by the fp32 and bf16 kernels: every address is
// clamped into its buffer, so the loads of the next K step issue as one
// straight-line block. Rows past M (columns past N) then repeat the last
// row (column): they only feed output rows (columns) that are never stored.
// Padded conv taps are zeroed.
#define GS_ROW_STATE()                                                                   \
  int arow[4];                                                                           \
  bool aval[4];                                                                          \
  /* implicit conv: top-left input coordinate of the row's window and the */          \
  /* offset of that (possibly padded) pixel's channel 0 */                               \
  int ohs[4], ows[4];                                                                    \
  int64_t cbase[4];                                                                      \
  float lnm[4], lnr[4]; /* A_LN: the row's mean and inv_std */                           \
  _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                        \
    const int m = m0 + lrow + 32 * i;                                                    \
    aval[i] = m < M;                                                                     \
    arow[i] = min(m, M - 1);                                                             \
    if (ALOAD == A_LN) {                                                                 \
      lnm[i] = p.ln_stats[2 * (int64_t)arow[i]];                                         \
      lnr[i] = p.ln_stats[2 * (int64_t)arow[i] + 1];                                     \
    }                                                                                    \
    if (ALOAD == A_CONV || ALOAD == A_CONV_H) {                                          \
      const int hw = p.cHo * p.cWo;                                                      \
      const int img = arow[i] / hw;                                                      \
      const int rem = arow[i] - img * hw;                                                \
      const int oh = rem / p.cWo, ow = rem - oh * p.cWo;                                 \
      ohs[i] = oh * p.cs - p.cp;                                                         \
      ows[i] = ow * p.cs - p.cp;                                                         \
      cbase[i] = (((int64_t)img * p.cH + ohs[i]) * p.cW + ows[i]) * p.cCin;              \
    }                                                                                    \
  }

// Origin of logical tile t of a problem. Grouped ordering: GROUP_M row tiles
// sweep the column tiles together, so consecutive tiles share A rows and B
// columns.
__device__ __forceinline__ void tile_mn(const GemmArgs& p, int t, int& m0, int& n0) {
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  const int per_group = GROUP_M * tiles_n;
  const int gid = t / per_group;
  const int first_m = gid * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  m0 = (first_m + (t % per_group) % gsz) * BM;
  n0 = ((t % per_group) / gsz) * BN;
}

// Tile coordinates of this workgroup (XCD-aware remap + grouped ordering);
// false when the workgroup has no tile in this group's problem.
__device__ __forceinline__ bool gemm_tile(const GemmArgs& p, int& m0, int& n0) {
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  const int ntiles = tiles_m * tiles_n;
  // Workgroups are dealt round-robin to the 8 XCDs; give each XCD a
  // contiguous range of logical tiles so neighbouring tiles (which share A
  // rows / B columns) meet in the same L2.
  int bid = blockIdx.x;
  const int nb = gridDim.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  if (bid >= ntiles) return false;
  tile_mn(p, bid, m0, n0);
  return true;
}

template <int ALOAD, int BLAYOUT, bool A_RELU>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmBatch batch) {
  const GemmArgs& p = batch.g[blockIdx.z];
  const int M = p.M, N = p.N, K = p.K;
  int m0, n0;
  if (!gemm_tile(p, m0, n0)) return;

  __shared__ __attribute__((aligned(16))) float As[BM][LDS];
  __shared__ __attribute__((aligned(16))) float Bs[BN][LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hl = lane >> 5;

  // Global->LDS assignment: rows tid/8 + 32*i, fx4 column tid%8.
  const int lrow = tid >> 3, lc4 = (tid & 7) * 4;

  GS_ROW_STATE()
  int boff[4];          // B row offsets (N * ldb < 2^31 is checked on the host)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (BLAYOUT == B_NT) {
      const int n = n0 + lrow + 32 * i;
      boff[i] = min(n, N - 1) * (int)p.ldb + lc4;
    }
  }
  int bncol = 0;
  if (BLAYOUT == B_NN) {
    const int n = n0 + 4 * (tid & 31);
    bncol = min(n, N - 4);
  }

  fx4 ra[4], rb[4], lgb[2];
  bool aok[4];
  const fx4 zero4 = mk4(0.f, 0.f, 0.f, 0.f);

  floatx16 acc00 = {}, acc01 = {}, acc10 = {}, acc11 = {};

  // The LayerNorm apply runs where its loads are issued (late in the MFMA
  // phase, where the compiler places them, so its VALU work hides under the
  // MFMAs); the conv zeroing and ReLU run at the LDS write (measured: each
  // placement is the faster one for its loader).
  constexpr bool fix_at_load = ALOAD == A_LN;
  // Where the next step's loads are issued among this step's 64 MFMAs, in
  // groups of 16 (4 = after all of them, placed by the compiler): measured
  // per loader on the model's shapes (conv 2 % and plain 2 % faster than at
  // the end; concat and LayerNorm best at the compiler's placement).
  constexpr int loadpos = ALOAD == A_CONV ? 3 : ALOAD == A_PLAIN ? 1 : 4;
  // split-K: this workgroup's contiguous K range (the whole K when ksplit == 1)
  int kbeg, kend;
  split_range(K, batch.ksplit, BK, kbeg, kend);
  GS_LOAD_A(kbeg)
  if (fix_at_load) GS_FIX_A()
  GS_LOAD_B_F32(kbeg)
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    __syncthreads();
    if (!fix_at_load) GS_FIX_A()
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *(fx4*)&As[lrow + 32 * i][lc4] = ra[i];
      if (BLAYOUT == B_NT) {
        *(fx4*)&Bs[lrow + 32 * i][lc4] = rb[i];
      } else {
        const int kb = (tid >> 5) + 8 * i;
        const int n = 4 * (tid & 31);
        Bs[n + 0][kb] = rb[i].x;
        Bs[n + 1][kb] = rb[i].y;
        Bs[n + 2][kb] = rb[i].z;
        Bs[n + 3][kb] = rb[i].w;
      }
    }
    __syncthreads();
    // Prefetch the next K step (the last iteration reloads its own step:
    // in bounds, and the values are never stored).
    if (loadpos >= 4) {
      GS_LOAD_A(min(k0 + BK, kend - BK))
      if (fix_at_load) GS_FIX_A()
      GS_LOAD_B_F32(min(k0 + BK, kend - BK))
    }
    const float* a0p = &As[wm * 64 + l32][hl * 16];
    const float* a1p = &As[wm * 64 + 32 + l32][hl * 16];
    const float* b0p = &Bs[wn * 64 + l32][hl * 16];
    const float* b1p = &Bs[wn * 64 + 32 + l32][hl * 16];
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) {
      const fx4 a0 = *(const fx4*)(a0p + t4 * 4);
      const fx4 a1 = *(const fx4*)(a1p + t4 * 4);
      const fx4 b0 = *(const fx4*)(b0p + t4 * 4);
      const fx4 b1 = *(const fx4*)(b1p + t4 * 4);
#define GS_MFMA4(AX, BX)                                                           \
  acc00 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.AX, b0.BX, acc00, 0, 0, 0);     \
  acc01 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.AX, b1.BX, acc01, 0, 0, 0);     \
  acc10 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.AX, b0.BX, acc10, 0, 0, 0);     \
  acc11 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.AX, b1.BX, acc11, 0, 0, 0);
      GS_MFMA4(x, x)
      GS_MFMA4(y, y)
      GS_MFMA4(z, z)
      GS_MFMA4(w, w)
#undef GS_MFMA4
      if (loadpos < 4 && t4 + 1 == loadpos) {
        __builtin_amdgcn_sched_barrier(0);
        GS_LOAD_A(min(k0 + BK, kend - BK))
        GS_LOAD_B_F32(min(k0 + BK, kend - BK))
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  if (batch.ksplit > 1)
    store_partial(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
  else
    gemm_epilogue(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
}


// Direct-to-LDS variant of the fp32 kernel for plain / concat A and NT B:
// global_load_lds_dwordx4 streams each K step straight into one of two LDS
// buffers (no VGPR staging, no ds_write), so the next step's tiles are in
// flight while the MFMAs consume the current one. LDS rows are 32 floats with
// the 16-byte chunks XOR-swizzled by row (chunk c of row r at slot
// c ^ ((r >> 1) & 7)): a wave's load instruction writes 8 contiguous rows
// (lane -> row lane>>3, slot lane&7). gfx950 LDS reads serve 16 lanes of
// 16 bytes per cycle from 64 banks, i.e. two 128-byte rows of banks; the MFMA
// reads of 16 consecutive rows at one chunk then hit 16 distinct bank groups
// (slot ^ (r & 7) left rows r and r + 8 on one group: 2-way conflicts,
// measured). Same per-element MFMA sequence as
// gemm_f32_kernel, so results are bit-identical to it. Synchronisation is
// explicit: s_waitcnt vmcnt leaves the next step's 8 loads in flight, and
// the barriers are bare s_barrier (a __syncthreads fence would also wait for
// the prefetch).
// LDS byte address of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_addr(const float* ptr) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)ptr;
}
// One wave-wide global_load_lds_dwordx4: lane l's 16 bytes at gptr land at
// LDS byte lds + 16*l (lds is wave-uniform, passed through M0). Issued as
// inline asm so that the compiler does not track it as an LDS store: its
// wait insertion cannot tell the two LDS buffers apart and would otherwise
// wait for the in-flight prefetch before every LDS read. The kernel waits
// for these loads itself (s_waitcnt vmcnt).
__device__ __forceinline__ void lds_dma16(const float* gptr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds), "v"(gptr)
               : "memory", "m0");
}

template <int ALOAD>
__global__ __launch_bounds__(256, 2) void gemm_f32_dl_kernel(GemmBatch batch) {
  const GemmArgs& p = batch.g[blockIdx.z];
  const int M = p.M, N = p.N;
  int m0, n0;
  if (!gemm_tile(p, m0, n0)) return;

  __shared__ __attribute__((aligned(16))) float As0[BM * BK];
  __shared__ __attribute__((aligned(16))) float Bs0[BN * BK];
  __shared__ __attribute__((aligned(16))) float As1[BM * BK];
  __shared__ __attribute__((aligned(16))) float Bs1[BN * BK];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hl = lane >> 5;

  // loader: wave w, instruction i fills tile rows 32w + 8i .. +7; the lane's
  // slot lane & 7 of row r holds chunk (lane & 7) ^ ((r >> 1) & 7)
  const int rin = lane >> 3;
  const float* ag[4];
  const float* ag2[4];
  const float* bg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 32 * wave + 8 * i + rin;
    const int chunk = (lane & 7) ^ ((row >> 1) & 7);
    const int64_t m = min(m0 + row, M - 1), n = min(n0 + row, N - 1);
    ag[i] = p.A + m * p.lda + 4 * chunk;
    ag2[i] = ALOAD == A_CONCAT ? p.A2 + m * p.lda2 + 4 * chunk - p.K1 : nullptr;
    bg[i] = p.B + n * p.ldb + 4 * chunk;
  }
#define GS_DL_ISSUE(BUF, K0)                                                            \
  {                                                                                     \
    const int k_ = (K0);                                                                \
    const bool first_ = ALOAD != A_CONCAT || k_ < p.K1;                                 \
    _Pragma("unroll") for (int i = 0; i < 4; ++i)                                       \
      lds_dma16((first_ ? ag[i] : ag2[i]) + k_, a_lds[BUF] + (32 * wave + 8 * i) * BK * 4); \
    _Pragma("unroll") for (int i = 0; i < 4; ++i)                                       \
      lds_dma16(bg[i] + k_, b_lds[BUF] + (32 * wave + 8 * i) * BK * 4);                 \
  }
  // per-lane LDS offsets of the MFMA operand rows; chunk c of row r sits at
  // slot c ^ ((r >> 1) & 7), the same for every operand row of the lane
  const int swz = (l32 >> 1) & 7;
  const int fa0 = (wm * 64 + l32) * BK, fa1 = fa0 + 32 * BK;
  const int fb0 = (wn * 64 + l32) * BK, fb1 = fb0 + 32 * BK;
  const uint32_t a_lds[2] = {lds_addr(As0), lds_addr(As1)};
  const uint32_t b_lds[2] = {lds_addr(Bs0), lds_addr(Bs1)};
#define GS_MFMA4(AX, BX)                                                           \
  acc00 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.AX, b0.BX, acc00, 0, 0, 0);     \
  acc01 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.AX, b1.BX, acc01, 0, 0, 0);     \
  acc10 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.AX, b0.BX, acc10, 0, 0, 0);     \
  acc11 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.AX, b1.BX, acc11, 0, 0, 0);
#define GS_DL_COMPUTE(AS, BS)                                                           \
  _Pragma("unroll") for (int t4 = 0; t4 < 4; ++t4) {                                    \
    const int co = ((hl * 4 + t4) ^ swz) << 2;                                          \
    const fx4 a0 = *(const fx4*)((AS) + fa0 + co);                                      \
    const fx4 a1 = *(const fx4*)((AS) + fa1 + co);                                      \
    const fx4 b0 = *(const fx4*)((BS) + fb0 + co);                                      \
    const fx4 b1 = *(const fx4*)((BS) + fb1 + co);                                      \
    GS_MFMA4(x, x)                                                                      \
    GS_MFMA4(y, y)                                                                      \
    GS_MFMA4(z, z)                                                                      \
    GS_MFMA4(w, w)                                                                      \
  }

  floatx16 acc00 = {}, acc01 = {}, acc10 = {}, acc11 = {};
  int kbeg, kend;
  split_range(p.K, batch.ksplit, BK, kbeg, kend);
  int k0 = kbeg;
  GS_DL_ISSUE(0, k0)
  while (true) {
    // K step k0 in buffer 0; step k0 + BK streams into buffer 1. Each wave
    // waits for its own 8 loads of step k0, then the barrier makes every
    // wave's loads visible; after the step every wave drains its LDS reads
    // (lgkmcnt(0)) before the barrier that lets buffer 0 be refilled.
    if (k0 + BK < kend) {
      GS_DL_ISSUE(1, k0 + BK)
      asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    }
    GS_DL_COMPUTE(As0, Bs0)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    k0 += BK;
    if (k0 >= kend) break;
    if (k0 + BK < kend) {
      GS_DL_ISSUE(0, k0 + BK)
      asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    }
    GS_DL_COMPUTE(As1, Bs1)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    k0 += BK;
    if (k0 >= kend) break;
  }
#undef GS_MFMA4
#undef GS_DL_ISSUE
#undef GS_DL_COMPUTE
  if (batch.ksplit > 1)
    store_partial(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
  else
    gemm_epilogue(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
}

// bf16-input / fp32-accumulate variant (v_mfma_f32_32x32x16_bf16): same tile,
// loaders and epilogue as the fp32 kernel; A is read in fp32 and rounded to
// bf16 (round-to-nearest-even) on its way into LDS, B is a bf16 copy of the
// weights ([N, K], NT layout). Within one K step of 32, MFMA slice s (0..1)
// feeds lane l (half h = l/32) with k = 16s + 8h .. 16s + 8h + 7, one
// ds_read_b128 per operand block. LDS rows hold 64 bf16 in swizzled order
// (bsw) for 64-deep steps, else 32 bf16 + 8 of padding.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
constexpr int LDSH = BK + 8;

// LDS rows of 64 bf16 (two 32-wide K chunks, 128 bytes, unpadded): the 8-byte
// chunk q of row r is stored at chunk q ^ bsw(r). On gfx950, LDS reads resolve
// 64 banks (16 lanes of 16 bytes per cycle) and writes 32 banks (16 lanes of
// 8 bytes, or 8 lanes of 16 bytes, per cycle). With this order, the fragment
// reads (16 rows, one 16-byte chunk each) and the staging writes (two rows per
// cycle) touch distinct banks. Padded rows of 72 conflicted 2-way on both
// operand writes.
__device__ __forceinline__ int bsw(int r) { return (((r >> 1) & 7) << 1) ^ ((r & 1) << 3); }
__device__ __forceinline__ int bsw_col(int col, int h) { return (((col >> 2) ^ h) << 2) | (col & 3); }

// KC: 32-wide K chunks per LDS step (2 where it divides the K range, else
// 1): one barrier pair then covers 8 KC MFMAs per wave. Each chunk is
// consumed in the order of a one-chunk step, so both give the same result.
// Measured on config 4 (bf16): two chunks 4 % faster per step than one (the
// linears 7 % faster); four chunks slower (69.6 KB of LDS, two workgroups
// per CU instead of three).
template <int ALOAD, bool A_RELU, int KC>
__global__ __launch_bounds__(256, 2) void gemm_bf16_kernel(GemmBatch batch) {
  constexpr int BLAYOUT = B_NT;
  // LDS row: two chunks swizzled (bsw), or one chunk + 8 bf16 of padding
  constexpr int LH = KC == 2 ? 2 * BK : BK + 8;
  static_assert(KC == 1 || KC == 2, "K chunks per step");
  const GemmArgs& p = batch.g[blockIdx.z];
  const int M = p.M, N = p.N, K = p.K;
  int m0, n0;
  if (!gemm_tile(p, m0, n0)) return;

  __shared__ __attribute__((aligned(16))) __bf16 As[BM][LH];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[BN][LH];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hl = lane >> 5;
  const int lrow = tid >> 3, lc4 = (tid & 7) * 4;

  GS_ROW_STATE()
  // B (bf16): rows tid/4 + 64*j (j < 2), 8 bf16 at column 8*(tid%4)
  const __bf16* Bh = (const __bf16*)p.Bh;
  const int brow = tid >> 2, bc8 = (tid & 3) * 8;
  // swizzle of the rows this thread writes (A: lrow + 32 i, B: brow + 64 j)
  // and reads (l32 + multiples of 32); 0 with padded single-chunk rows
  const int hA = KC == 2 ? bsw(lrow) : 0, hB = KC == 2 ? bsw(brow) : 0;
  const int hR = KC == 2 ? bsw(l32) : 0;
  int bo[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + brow + 64 * j;
    bo[j] = min(n, N - 1) * (int)p.ldb + bc8;
  }

  // register stage per chunk: fp32 A (fixed up and converted at the store)
  // or bf16 A (A_PLAIN_H, stored as loaded), and bf16 B
  fx4 rac[KC][4], lgbc[KC][2];
  bool aokc[KC][4];
  bf16x4 rahc[KC][4];
  bf16x8 rbhc[KC][2];
  const fx4 zero4 = mk4(0.f, 0.f, 0.f, 0.f);

  floatx16 acc00 = {}, acc01 = {}, acc10 = {}, acc11 = {};

#define GS_LOAD_AH(K0, C)                                                        \
  {                                                                              \
    fx4* const ra = rac[C];                                                      \
    fx4* const lgb = lgbc[C];                                                    \
    bool* const aok = aokc[C];                                                   \
    (void)ra;                                                                    \
    (void)lgb;                                                                   \
    (void)aok;                                                                   \
    if (ALOAD == A_PLAIN_H) {                                                    \
      const __bf16* Ah = (const __bf16*)p.A;                                     \
      _Pragma("unroll") for (int i = 0; i < 4; ++i)                              \
        rahc[C][i] = *(const bf16x4*)(Ah + (int64_t)arow[i] * p.lda + (K0) + lc4); \
    } else if (ALOAD == A_CONV_H) {                                              \
      /* bf16 NHWC input: tap (kh, kw), channels ic0..; padded taps read */      \
      /* element lc4 (in bounds) and are zeroed at the LDS write */              \
      const __bf16* Ah = (const __bf16*)p.A;                                     \
      const int kk = (K0) / p.cCin;                                              \
      const int ic0 = (K0) - kk * p.cCin;                                        \
      const int kh = kk / p.ckw, kw = kk - kh * p.ckw;                             \
      const int64_t toff = ((int64_t)kh * p.cW + kw) * p.cCin + ic0;             \
      _Pragma("unroll") for (int i = 0; i < 4; ++i) {                            \
        const int ih = ohs[i] + kh, iw = ows[i] + kw;                            \
        const bool ok = aval[i] && (unsigned)ih < (unsigned)p.cH &&               \
                        (unsigned)iw < (unsigned)p.cW;                           \
        aok[i] = ok;                                                             \
        rahc[C][i] = *(const bf16x4*)(Ah + (ok ? cbase[i] + toff : 0) + lc4);     \
      }                                                                          \
    } else {                                                                     \
      GS_LOAD_A(K0)                                                              \
    }                                                                            \
  }
#define GS_LOAD_B_BF16(K0, C)                                                    \
  _Pragma("unroll") for (int j = 0; j < 2; ++j)                                  \
    rbhc[C][j] = *(const bf16x8*)(Bh + bo[j] + (K0));
#define GS_LOAD_STEP(K0)                                                         \
  _Pragma("unroll") for (int c = 0; c < KC; ++c) {                               \
    GS_LOAD_AH((K0) + BK * c, c)                                                 \
    GS_LOAD_B_BF16((K0) + BK * c, c)                                             \
  }

  constexpr int SK = BK * KC;
  // Where the next step's loads are issued among this step's 2 KC groups of
  // four MFMAs (0 = before the first): measured per loader at config 4
  // (plain rows after the first group: fp32 rows 14 %, bf16 rows 1 % faster;
  // conv after the third, concat before the first). Clamped to the last
  // group, so every step issues its prefetch.
  constexpr int lp_want = (ALOAD == A_CONV || ALOAD == A_CONV_H) ? 3
                         : (ALOAD == A_PLAIN || ALOAD == A_PLAIN_H) ? 1 : 0;
  constexpr int loadpos = lp_want < 2 * KC ? lp_want : 2 * KC - 1;
  int kbeg, kend;
  split_range(K, batch.ksplit, SK, kbeg, kend);
  GS_LOAD_STEP(kbeg)
  for (int k0 = kbeg; k0 < kend; k0 += SK) {
    __syncthreads();
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      fx4* const ra = rac[c];
      const fx4* const lgb = lgbc[c];
      const bool* const aok = aokc[c];
      (void)lgb;
      (void)aok;
      if (ALOAD != A_PLAIN_H && ALOAD != A_CONV_H) GS_FIX_A()
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16x4 h;
        if (ALOAD == A_PLAIN_H) {
          h = rahc[c][i];
        } else if (ALOAD == A_CONV_H) {
          const bf16x4 z = {};
          h = aok[i] ? rahc[c][i] : z;  // padded tap
        } else {
          h.x = (__bf16)ra[i].x;
          h.y = (__bf16)ra[i].y;
          h.z = (__bf16)ra[i].z;
          h.w = (__bf16)ra[i].w;
        }
        *(bf16x4*)&As[lrow + 32 * i][bsw_col(BK * c + lc4, hA)] = h;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) *(bf16x8*)&Bs[brow + 64 * j][bsw_col(BK * c + bc8, hB)] = rbhc[c][j];
    }
    __syncthreads();
    if (loadpos == 0) GS_LOAD_STEP(min(k0 + SK, kend - SK))
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      if (loadpos > 0 && 2 * c + sl == loadpos) {
        __builtin_amdgcn_sched_barrier(0);
        GS_LOAD_STEP(min(k0 + SK, kend - SK))
        __builtin_amdgcn_sched_barrier(0);
      }
      const int kc = bsw_col(BK * c + sl * 16 + hl * 8, hR);
      const bf16x8 a0 = *(const bf16x8*)&As[wm * 64 + l32][kc];
      const bf16x8 a1 = *(const bf16x8*)&As[wm * 64 + 32 + l32][kc];
      const bf16x8 b0 = *(const bf16x8*)&Bs[wn * 64 + l32][kc];
      const bf16x8 b1 = *(const bf16x8*)&Bs[wn * 64 + 32 + l32][kc];
      acc00 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc00, 0, 0, 0);
      acc01 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc01, 0, 0, 0);
      acc10 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc10, 0, 0, 0);
      acc11 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc11, 0, 0, 0);
    }
  }
#undef GS_LOAD_STEP
#undef GS_LOAD_B_BF16
#undef GS_LOAD_AH
  if (batch.ksplit > 1)
    store_partial(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
  else
    gemm_epilogue(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
}

// fp32 GEMM through bf16 matrix cores ("bf16x6"): every fp32 operand x is
// split exactly into three bf16 terms x = x0 + x1 + x2 (x0 = bf16(x),
// x1 = bf16(x - x0), x2 = bf16(x - x0 - x1); each remainder is exact in fp32)
// and the product is accumulated in fp32 from the six term products whose
// relative size is at least 2^-16 (x0y0, x0y1, x1y0, x1y1, x0y2, x2y0; the
// dropped x1y2, x2y1, x2y2 are <= 2^-24 relative, the size of one fp32
// rounding). Each bf16 x bf16 product is exact in the fp32 accumulation, so
// the result has fp32-level accuracy at 6 bf16 MFMAs (32 cycles each) per
// 32x32x16 block instead of 8 fp32 MFMAs (64 cycles each). Same tile,
// loaders (plain / concat / conv, ReLU prologue) and epilogue as
// gemm_f32_kernel; operands are read in fp32 and split on their way into
// LDS, three bf16 planes per operand.
// BSPLIT: B arrives pre-split (planes at Bh + t * bh_plane, same arithmetic,
// so the products are bit-identical) and is copied into LDS as loaded.
// Terms are accumulated smallest first.
__device__ __forceinline__ void split3(const fx4& v, bf16x4& h, bf16x4& m, bf16x4& l) {
  uint32_t h0, m0, l0, h1, m1, l1;
  split3_pk(v.x, v.y, h0, m0, l0);
  split3_pk(v.z, v.w, h1, m1, l1);
  h = __builtin_bit_cast(bf16x4, (uint64_t)h0 | ((uint64_t)h1 << 32));
  m = __builtin_bit_cast(bf16x4, (uint64_t)m0 | ((uint64_t)m1 << 32));
  l = __builtin_bit_cast(bf16x4, (uint64_t)l0 | ((uint64_t)l1 << 32));
}

// bf16-input / fp32-accumulate kernel for large launches with bf16 activations
// (A_PLAIN_H) and NT bf16 weights: workgroup tile 256 x 128 of 2 x 2 waves at
// 128 x 64 (4 x 2 MFMA 32x32x16 blocks, 128 accumulators per lane), 32-deep K
// steps streamed straight into one of two LDS stages (global_load_lds_dwordx4,
// 48 KB in all), two or three workgroups per CU. Each wave reads 6 fragments
// per 8 MFMAs (the 128 x 128 kernel: 4 per 4), and with more than one
// workgroup per CU one workgroup's epilogue runs under the others' MFMAs,
// which a 256 x 256 tile at one workgroup per CU cannot do.
// LDS rows are 32 bf16 (64 bytes, four 16-byte chunks); a load instruction
// fills 16 rows (lane -> row lane >> 2, slot lane & 3), and chunk c of row r
// sits at slot c ^ ((r >> 2) & 3): four rows share a 256-byte bank line, so
// the fragment reads of 16 consecutive rows at one chunk hit 16 distinct bank
// groups. Lane l (half h) feeds slice s with k = 16s + 8h .. +7: the
// per-element MFMA sequence of gemm_bf16_kernel. The accumulators go out
// through w2_epi_row, one 32-row block row at a time.
constexpr int W2M = 256, W2N = 128, W2K = 32;
constexpr int W2_STAGE = (W2M + W2N) * W2K;  // bf16 per LDS stage
constexpr int W2_SS = 68;                    // epilogue stage row stride (floats)
constexpr int W2_SS1 = 36;                   // the same for one 32-column block
// fp32 256 x 128 kernel dispatch: at least this many tiles, one full round at
// three workgroups per CU (measured at config 3: the 576-tile decoder launches
// run 105 TFLOP/s on it against 120 on the 128 x 128 kernels)
constexpr int kF2MinTiles = 768;
// Small launches (plain rows below one round of 256 x 128 tiles, implicit
// convs below one round of 192 x 128) take the 64-row form unsplit from this
// many of its tiles. Measured against the split 128 x 128 kernel at one image
// / one pair: 432 tiles (decoder qkv, two chains) +5 %, 576 +0-5 %, 768
// (encoder fc1 on two images) +8 %; 288 and 384 tiles 10-20 % slower. The
// 2304-deep DPT convs of 768 tiles: 120-123 TFLOP/s against 116 for the
// register-staged conv split in two.
constexpr int kW64MinTiles = 432;
// Plain-row launches too small for that take the 32-row form (1 x 4 waves at
// 32 x 32) unsplit from this many of its tiles: three per CU (one image's
// encoder fc1, M = 768 and N = 4096: 100 TFLOP/s with no reduce pass, against
// 91 for the 128 x 128 kernel split in four; at 576 tiles, one image's qkv,
// it ran level with the split kernel and the encoder 0.4 % slower than at
// this threshold). It also takes launches of the 64-row form whose busiest
// CU it loads less (one pair: the encoder qkv, 576 tiles of 64 rows, 3 per
// CU, against 1152 of 32 rows, 5 per CU: 91.5 -> 97.7 TFLOP/s; the decoder
// fc1 88.4 -> 96.4), and smaller launches whose busiest CU it loads no more
// than the split 128 x 128 kernel does and which write no LayerNorm (the
// short-K launches at one pair: K = 96, M = 768 and N = 1536, 11.5 -> 31
// TFLOP/s; the encoder proj, M = 1536, N = 1024, K = 1024, ran 62.2 -> 69.9
// but then needed its LayerNorm pass back, 0.18 ms per pair; at K = 4096 the
// split kernel's three 512-deep ranges per CU beat two full 32-row tiles,
// 103 against 81 TFLOP/s). Launches of 512-767 tiles that write no
// LayerNorm run it split in K (one image's qkv, 576 tiles in three ranges:
// 62 -> 58 us against the split 128 x 128 kernel; the LayerNorm-writing proj
// and fc2 ran 1-40 % slower split this way).
constexpr int kW32MinTiles = 768;
// Long-K launches of the fp32 256 x 128 kernel run as one launch per round of
// workgroup slots (96 tiles per XCD: 32 CUs x 3 workgroups), so every round
// starts together, as the first round of one launch does, and its tiles stream
// their shared A / B panels through the XCD's L2 at the same K; across the later
// rounds of one launch the tiles drift apart and each re-fetches its panels
constexpr int kF2PhaseMinK = 6144, kF2PhaseTiles = 96;
static_assert(4 * 32 * W2_SS * 4 <= 2 * W2_STAGE * 2, "w2 epilogue stages fit the LDS stages");

// Epilogue of one 32 x 64 block row of a gemm_bf16_w2_kernel wave (q0: columns
// col0 .. +31, q1: col0 + 32 .. +63): bias, RoPE, GELU / ReLU on the
// accumulators, then through the wave's LDS stage (32 rows of W2_SS floats) so
// that residuals are read and outputs written as 16-byte row segments (16
// lanes per 64-column row). Same per-element operations and order as
// gemm_epilogue_t. The scatter form (ConvT / pixel shuffle) stores 4-column
// segments, each inside one output pixel: the host admits it only with
// sc_C % 4 == 0, sc_Cout % 4 == 0 and no residual, RoPE or dual store
// (row_epi_ok). Measured in the
// model: the per-element form of the shared epilogue (64-bit addresses, 4-byte
// accesses) took this kernel from ~1100 TFLOP/s (main loop) to 360-565.
template <bool ROPE, int NB = 2>
__device__ __forceinline__ void w2_epi_row(const GemmArgs& p, const floatx16& q0,
                                           const floatx16& q1, int row0, int col0, float* stage,
                                           int lane, int l32, int hl) {
  static_assert(NB == 1 || NB == 2, "one or two 32-column blocks");
  constexpr int SS = NB == 2 ? W2_SS : W2_SS1;  // stage row stride (floats)
  const int M = p.M, N = p.N;
  const int flags = ROPE ? p.flags & ~(EPI_RES1 | EPI_RES2) : p.flags & ~EPI_ROPE;
  const float rtok = ROPE ? 1.0f / (float)p.tok_per_img : 0.f;
  const float rgw = ROPE ? 1.0f / (float)p.grid_w : 0.f;
  // NB = 2: col0 is a multiple of 64, so q0 is the y-axis half and q1 the
  // x-axis half of one head's RoPE columns. NB = 1 (one 32-column block, q1
  // unused): col0 is a multiple of 32 and names the half
  const float bv0 = (flags & EPI_BIAS) ? p.bias[min(col0 + l32, N - 1)] : 0.f;
  const float bv1 =
      (NB == 2 && (flags & EPI_BIAS)) ? p.bias[min(col0 + 32 + l32, N - 1)] : 0.f;
  const bool rope = ROPE && col0 < p.rope_ncols;
  const bool xhalf = NB == 1 && (col0 & 32) != 0;
  // With the tokens per image and the grid width multiples of 4, the four
  // rows 4k .. 4k + 3 of accumulator registers 4g .. 4g + 3 lie in one image
  // and grid row: their position is decoded once (the first row's, x + j for
  // row j) and the y-axis cos / sin are read once. Rows at or past M are not
  // stored; their group decodes the last group start below M.
  const bool grp4 = ROPE && ((p.tok_per_img | p.grid_w) & 3) == 0;
  int gty = 0, gtx = 0;
  float gcy = 0.f, gsy = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float v0 = q0[r], v1 = q1[r];
    if (flags & EPI_BIAS) {
      v0 = v0 + bv0;
      v1 = v1 + bv1;
    }
    if (rope) {
      // the row's grid position, frequency l32 % 16
      int ty, tx;
      float cy, sy;
      if (grp4) {
        if ((r & 3) == 0) {
          const int rg = min(row0 + 8 * (r >> 2) + 4 * hl, (M - 1) & ~3);
          int tok;
          divmod_small(rg, p.tok_per_img, rtok, tok);
          gty = divmod_small(tok, p.grid_w, rgw, gtx);
          const int iy = gty * 16 + (l32 & 15);
          gcy = p.rope_cos[iy];
          gsy = p.rope_sin[iy];
        }
        ty = gty;
        tx = gtx + (r & 3);
        cy = gcy;
        sy = gsy;
      } else {
        const int row = min(row0 + 8 * (r >> 2) + 4 * hl + (r & 3), M - 1);
        int tok;
        divmod_small(row, p.tok_per_img, rtok, tok);
        ty = divmod_small(tok, p.grid_w, rgw, tx);
        const int iy = ty * 16 + (l32 & 15);
        cy = p.rope_cos[iy];
        sy = p.rope_sin[iy];
      }
      (void)ty;
      const int ix = tx * 16 + (l32 & 15);
      const float cx = p.rope_cos[ix], sx = p.rope_sin[ix];
      if constexpr (NB == 2) {
        const float p0 = __shfl_xor(v0, 16), p1 = __shfl_xor(v1, 16);
        v0 = (l32 < 16) ? (v0 * cy - p0 * sy) : (v0 * cy + p0 * sy);
        v1 = (l32 < 16) ? (v1 * cx - p1 * sx) : (v1 * cx + p1 * sx);
      } else {
        const float c = xhalf ? cx : cy, sn = xhalf ? sx : sy;
        const float p0 = __shfl_xor(v0, 16);
        v0 = (l32 < 16) ? (v0 * c - p0 * sn) : (v0 * c + p0 * sn);
      }
    }
    if (flags & EPI_GELU) {
      v0 = gelu_tanh(v0);
      v1 = gelu_tanh(v1);
    }
    if (flags & EPI_RELU) {
      v0 = fmaxf(v0, 0.f);
      v1 = fmaxf(v1, 0.f);
    }
    float* srow = stage + (8 * (r >> 2) + 4 * hl + (r & 3)) * SS + l32;
    srow[0] = v0;
    if constexpr (NB == 2) srow[32] = v1;
  }
  // the stage belongs to this wave: LDS accesses of one wave complete in
  // order, so a wave-level fence orders the writes above and the reads below
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // readback: LPR lanes per row (4 columns each), RPP rows per pass, UPH
  // passes per 16-row half
  constexpr int LPR = 8 * NB, RPP = 64 / LPR, UPH = 16 / RPP;
  const int rin = lane / LPR, c4 = (lane % LPR) * 4;
  const int col = col0 + c4;
  const int colc = min(col, N - 4);
  // sub-pixel scatter (EPI_SCATTER): column col = (i * sc_r + j) * sc_C + c;
  // with sc_C and sc_Cout multiples of 4 the lane's 4 columns are one pixel's
  // channels c .. c + 3, all kept or all dropped, 16 contiguous output bytes
  int sc_i = 0, sc_j = 0, sc_c = 0;
  if (flags & EPI_SCATTER) {
    const int sidx = col / p.sc_C;
    sc_c = col - sidx * p.sc_C;
    sc_i = sidx / p.sc_r;
    sc_j = sidx - sc_i * p.sc_r;
  }
  // two halves of 16 rows, the residuals of a half read before its stores
#pragma unroll
  for (int hq = 0; hq < 2; ++hq) {
  fx4 x1[UPH], x2[UPH];
  if (flags & EPI_RES1) {
#pragma unroll
    for (int u = 0; u < UPH; ++u) {
      const int row = min(row0 + 16 * hq + RPP * u + rin, M - 1);
      x1[u] = *(const fx4*)(p.R1 + (int64_t)row * p.ldr1 + colc);
    }
  }
  if (flags & EPI_RES2) {
#pragma unroll
    for (int u = 0; u < UPH; ++u) {
      const int row = min(row0 + 16 * hq + RPP * u + rin, M - 1);
      x2[u] = *(const fx4*)(p.R2 + (int64_t)row * p.ldr2 + colc);
    }
  }
#pragma unroll
  for (int u = 0; u < UPH; ++u) {
    const int sr = 16 * hq + RPP * u + rin;
    const int row = row0 + sr;
    fx4 v = *(const fx4*)(stage + sr * SS + c4);
    if (flags & EPI_RES1) v = v + x1[u];
    if (flags & EPI_RES2) v = x2[u] + v;
    if (row < M && col < N) {
      if (flags & EPI_SCATTER) {
        if (sc_c < p.sc_Cout) {
          const int hw = p.sc_gh * p.sc_gw;
          const int img = row / hw;
          const int rem = row - img * hw;
          const int yy = rem / p.sc_gw, xx = rem - yy * p.sc_gw;
          const int64_t oy = (int64_t)img * p.sc_gh * p.sc_r + yy * p.sc_r + sc_i;
          const int64_t ox = (int64_t)xx * p.sc_r + sc_j;
          const int64_t si = (oy * p.sc_gw * p.sc_r + ox) * p.sc_Cout + sc_c;
          if (flags & EPI_BF16OUT) {
            typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
            const bf16x4_t h = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
            *(bf16x4_t*)((__bf16*)p.C + si) = h;
          } else {
            *(fx4*)(p.C + si) = v;
          }
        }
      } else if (flags & EPI_BF16OUT) {
        typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
        bf16x4_t h;
        h.x = (__bf16)v.x;
        h.y = (__bf16)v.y;
        h.z = (__bf16)v.z;
        h.w = (__bf16)v.w;
        *(bf16x4_t*)((__bf16*)p.C + (int64_t)row * p.ldc + col) = h;
      } else {
        *(fx4*)(p.C + (int64_t)row * p.ldc + col) = v;
        if (flags & EPI_DUAL) dual_store(p, flags, (int64_t)row * p.ldc + col, v);
      }
    }
  }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int BM>
__device__ __forceinline__ bool f2_tile(const GemmBatch& batch, const GemmArgs& p, int& m0,
                                        int& n0) {
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + W2N - 1) / W2N;
  const int ntiles = tiles_m * tiles_n;
  int bid = blockIdx.x;
  const int nb = gridDim.x;
  if (batch.tphase_q)
    bid = (bid & 7) * batch.tphase_q + batch.tphase_base + (bid >> 3);
  else if ((nb & 7) == 0)
    bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  if (bid >= ntiles) return false;
  const int per_group = GROUP_M * tiles_n;
  const int gid = bid / per_group;
  const int first_m = gid * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  m0 = (first_m + (bid % per_group) % gsz) * BM;
  n0 = ((bid % per_group) / gsz) * W2N;
  return true;
}

// 64 zero bytes: the source of a padded conv tap's 16-byte loads
__device__ __attribute__((aligned(64))) float g_zero16[16] = {};

// plain-row launches with at least this K per group take the three-stage
// form (measured at config 4: descriptor fc2, K = 7168, 695 -> 832 TFLOP/s;
// encoder fc2, K = 4096, 872 / 865; K <= 1024 linears and the implicit convs
// 7-13 % slower, their epilogues exposed at two workgroups per CU)
constexpr int kW2ThreeStageMinK = 6144;

// BM = 256 or 192 rows; CONV: the A rows gathered from a bf16 NHWC input
// (implicit conv, A_CONV_H; a 32-deep K step is 32 channels of one tap, so a
// lane's 16 bytes are contiguous; padded taps load from g_zero16).
// NST = 2: two LDS stages, three workgroups per CU, loads issued one K step
// ahead, two barriers per step. NST = 3: three stages, two workgroups per CU,
// loads issued two steps ahead and one barrier per step (the barrier that
// makes step k visible also retires every wave's reads of step k - 1, whose
// stage the loads of step k + 2 then refill).
template <int BM, bool CONV, int NST>
__global__ __launch_bounds__(256, NST == 3 ? 2 : 3) void gemm_bf16_w2_kernel(GemmBatch batch) {
  constexpr int WTM = BM / 64;                 // 32-row blocks per wave
  constexpr int BSTAGE = (BM + W2N) * W2K;     // bf16 per LDS stage
  constexpr int LPS = BM / 64 + W2N / 64;      // loads per wave per K step
  static_assert(BM == 256 || BM == 192, "tile rows");
  static_assert(NST == 2 || NST == 3, "LDS stages");
  static_assert(4 * 32 * W2_SS * 4 <= NST * BSTAGE * 2, "w2 epilogue stages fit the LDS stages");
  const GemmArgs& p = batch.g[blockIdx.z];
  const int M = p.M, N = p.N, K = p.K;
  int m0, n0;
  if (!f2_tile<BM>(batch, p, m0, n0)) return;
  __shared__ __attribute__((aligned(16))) __bf16 lds[NST * BSTAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hl = lane >> 5;
  // loader: wave w, instruction i fills tile rows 16 (4i + w) .. +15; the
  // slot swizzle (r >> 2) & 3 of those rows is (rin >> 2) & 3 for every i
  const int rin = lane >> 2, chunk = (lane & 3) ^ ((rin >> 2) & 3);
  const __bf16* Ah = (const __bf16*)p.A;
  const __bf16* Bh = (const __bf16*)p.Bh;
  const __bf16* ag[BM / 64];
  const __bf16* bg[W2N / 64];
  int ohs[BM / 64], ows[BM / 64];
#pragma unroll
  for (int i = 0; i < BM / 64; ++i) {
    const int mr = m0 + 16 * (4 * i + wave) + rin;
    const int64_t m = min(mr, M - 1);
    if constexpr (CONV) {
      const int hw = p.cHo * p.cWo;
      const int img = (int)(m / hw), rem = (int)(m - (int64_t)img * hw);
      const int oh = rem / p.cWo, ow = rem - oh * p.cWo;
      const int ih0 = oh * p.cs - p.cp;
      ows[i] = ow * p.cs - p.cp;
      ag[i] = Ah + (((int64_t)img * p.cH + ih0) * p.cW + ows[i]) * p.cCin + 8 * chunk;
      ohs[i] = mr < M ? ih0 : -(1 << 20);  // rows past M: never in bounds
    } else {
      ag[i] = Ah + m * p.lda + 8 * chunk;
    }
  }
#pragma unroll
  for (int i = 0; i < W2N / 64; ++i) {
    const int64_t n = min(n0 + 16 * (4 * i + wave) + rin, N - 1);
    bg[i] = Bh + n * p.ldb + 8 * chunk;
  }
  const uint32_t lds0 = lds_addr((const float*)lds);
  // conv tap state of the next step to issue (wave-uniform)
  int tkh = 0, tkw = 0, tic = 0;
  const float* zrow = g_zero16 + 4 * chunk;
#define GS_W2_ISSUE(BUF, K0)                                                                 \
  {                                                                                          \
    if constexpr (CONV) {                                                                    \
      const int64_t toff = ((int64_t)tkh * p.cW + tkw) * p.cCin + tic;                       \
      _Pragma("unroll") for (int i = 0; i < BM / 64; ++i) {                                  \
        const bool ok = (unsigned)(ohs[i] + tkh) < (unsigned)p.cH &&                          \
                        (unsigned)(ows[i] + tkw) < (unsigned)p.cW;                            \
        lds_dma16(ok ? (const float*)(ag[i] + toff) : zrow,                                  \
                  lds0 + ((BUF) * BSTAGE + 16 * (4 * i + wave) * W2K) * 2);                  \
      }                                                                                      \
      tic += W2K;                                                                            \
      if (tic == p.cCin) {                                                                   \
        tic = 0;                                                                             \
        if (++tkw == p.ckw) {                                                                 \
          tkw = 0;                                                                           \
          ++tkh;                                                                             \
        }                                                                                    \
      }                                                                                      \
    } else {                                                                                 \
      _Pragma("unroll") for (int i = 0; i < BM / 64; ++i)                                    \
        lds_dma16((const float*)(ag[i] + (K0)),                                              \
                  lds0 + ((BUF) * BSTAGE + 16 * (4 * i + wave) * W2K) * 2);                  \
    }                                                                                        \
    _Pragma("unroll") for (int i = 0; i < W2N / 64; ++i)                                     \
      lds_dma16((const float*)(bg[i] + (K0)),                                                \
                lds0 + ((BUF) * BSTAGE + (BM + 16 * (4 * i + wave)) * W2K) * 2);             \
  }
  const int swz = (l32 >> 2) & 3;
  const int ra0 = (wm * 32 * WTM + l32) * W2K, rb0 = (wn * 64 + l32) * W2K;
  floatx16 c00 = {}, c01 = {}, c10 = {}, c11 = {}, c20 = {}, c21 = {}, c30 = {}, c31 = {};
  int buf = 0;
  GS_W2_ISSUE(0, 0)
  if (NST == 3 && W2K < K) GS_W2_ISSUE(1, W2K)
  for (int k0 = 0; k0 < K; k0 += W2K) {
    if constexpr (NST == 2) {
      // step k0 in stage buf, step k0 + W2K streaming into the other stage:
      // each wave waits for its own LPS loads of step k0, the barrier makes
      // all of them visible; the fragment reads drain before the barrier
      // that lets the stage be refilled
      if (k0 + W2K < K) {
        GS_W2_ISSUE(buf ^ 1, k0 + W2K)
        if constexpr (BM == 256)
          asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
        else
          asm volatile("s_waitcnt vmcnt(5)\n\ts_barrier" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      }
    } else {
      // steps k0 and k0 + W2K in flight: wait for this wave's loads of step
      // k0 (the LPS loads of step k0 + W2K may stay outstanding) and for its
      // reads of step k0 - W2K; after the barrier every wave's loads of step
      // k0 are visible and no wave reads the stage of step k0 - W2K, which
      // the loads of step k0 + 2 W2K refill
      static_assert(LPS == 6 || LPS == 5, "vmcnt immediates below");
      if (k0 + W2K < K) {
        if constexpr (LPS == 6)
          asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else
          asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
      if (k0 + 2 * W2K < K) GS_W2_ISSUE(buf == 0 ? 2 : buf - 1, k0 + 2 * W2K)
    }
    const __bf16* as = lds + buf * BSTAGE;
    const __bf16* bs = as + BM * W2K;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int co = ((2 * s + hl) ^ swz) << 3;
      const bf16x8 a0 = *(const bf16x8*)(as + ra0 + co);
      const bf16x8 a1 = *(const bf16x8*)(as + ra0 + 32 * W2K + co);
      const bf16x8 a2 = *(const bf16x8*)(as + ra0 + 64 * W2K + co);
      bf16x8 a3 = {};
      if constexpr (WTM == 4) a3 = *(const bf16x8*)(as + ra0 + 96 * W2K + co);
      const bf16x8 b0 = *(const bf16x8*)(bs + rb0 + co);
      const bf16x8 b1 = *(const bf16x8*)(bs + rb0 + 32 * W2K + co);
      c00 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, c00, 0, 0, 0);
      c01 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, c01, 0, 0, 0);
      c10 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, c10, 0, 0, 0);
      c11 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, c11, 0, 0, 0);
      c20 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b0, c20, 0, 0, 0);
      c21 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b1, c21, 0, 0, 0);
      if constexpr (WTM == 4) {
        c30 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a3, b0, c30, 0, 0, 0);
        c31 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a3, b1, c31, 0, 0, 0);
      }
    }
    if constexpr (NST == 2) {
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      buf ^= 1;
    } else {
      buf = buf == 2 ? 0 : buf + 1;
    }
  }
  // the epilogue stages overlay the LDS stages: every wave's last reads first
  if constexpr (NST == 3) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#undef GS_W2_ISSUE
  // WTM 32-row block rows per wave through the staged epilogue (the wave's
  // 32 x 68-float stage; the LDS stages are free after the last barrier)
  const int mw = m0 + wm * 32 * WTM, nw = n0 + wn * 64;
  float* stage = (float*)lds + wave * 32 * W2_SS;
  if (p.flags & EPI_ROPE) {
    w2_epi_row<true>(p, c00, c01, mw, nw, stage, lane, l32, hl);
    w2_epi_row<true>(p, c10, c11, mw + 32, nw, stage, lane, l32, hl);
    w2_epi_row<true>(p, c20, c21, mw + 64, nw, stage, lane, l32, hl);
    if constexpr (WTM == 4) w2_epi_row<true>(p, c30, c31, mw + 96, nw, stage, lane, l32, hl);
  } else {
    w2_epi_row<false>(p, c00, c01, mw, nw, stage, lane, l32, hl);
    w2_epi_row<false>(p, c10, c11, mw + 32, nw, stage, lane, l32, hl);
    w2_epi_row<false>(p, c20, c21, mw + 64, nw, stage, lane, l32, hl);
    if constexpr (WTM == 4) w2_epi_row<false>(p, c30, c31, mw + 96, nw, stage, lane, l32, hl);
  }
}

// fp32 kernel of the same structure for large launches with plain rows or an
// implicit conv (CONV: each K step's A rows gathered from the NHWC input, see
// below):
// workgroup tile BM x 128 (BM = 256, 192 or 64) of 2 x 2 waves at (BM / 2) x 64
// (BM / 64 x 2 blocks of v_mfma_f32_32x32x2_f32), 16-deep K steps (64-byte
// rows: the bf16 kernel's LDS geometry, loader and slot swizzle) streamed into
// two LDS stages (48 / 40 KB; 35 KB at BM = 64 and 32, where the epilogue
// stages are larger than the K stages), three workgroups per CU (four at
// BM = 64),
// epilogue through w2_epi_row. Lane l (half h) feeds MFMA step t of a K step
// with k = 8h + t. BM = 192 serves launches whose 256-row tiles would leave
// part of the last round of workgroup slots empty (the decoder's N = 768
// linears: 576 tiles of 256 rows on 768 slots, exactly 768 of 192 rows);
// BM = 64 serves launches below one round of 256-row tiles (convs: of
// 192-row tiles) that make at least kW64MinTiles of its tiles, without
// split-K. BM = 32 (plain rows) serves smaller launches that still make
// kW32MinTiles of its tiles: 1 x 4 waves at 32 x 32 (one MFMA block each);
// the 32 A rows of a K step are two waves' loads, and waves 2 and 3 issue
// the same two loads again (identical bytes to the same LDS words), so every
// wave issues three loads per K step, as at BM = 64. Split launches give each
// blockIdx.y one K range and store its raw partial for gemm_splitk_reduce.


template <int BM, bool CONV>
__global__ __launch_bounds__(256, 3) void gemm_f32_w2_kernel(GemmBatch batch) {
  constexpr int FK = 16;                     // floats per K step
  constexpr bool W1X4 = BM == 32;            // 1 x 4 waves at 32 x 32
  constexpr int WTM = W1X4 ? 1 : BM / 64;    // 32-row blocks per wave
  constexpr int NA = W1X4 ? 1 : BM / 64;     // A-row loads per wave per K step
  constexpr int FSTAGE = (BM + W2N) * FK;    // floats per LDS stage
  // the epilogue's four 32-row wave stages overlay the LDS stages (BM = 64
  // allocates past the two K stages for them; BM = 32, one 32-column block
  // per wave, fits in them: 20 KB, so up to eight workgroups per CU)
  constexpr int ESTAGE = 4 * 32 * (W1X4 ? W2_SS1 : W2_SS);  // the four wave stages
  constexpr int LDSF = 2 * FSTAGE > ESTAGE ? 2 * FSTAGE : ESTAGE;
  static_assert(BM == 256 || BM == 192 || BM == 64 || (BM == 32 && !CONV), "tile rows");
  const GemmArgs& p = batch.g[blockIdx.z];
  const int M = p.M, N = p.N, K = p.K;
  int m0, n0;
  if (!f2_tile<BM>(batch, p, m0, n0)) return;
  __shared__ __attribute__((aligned(16))) float lds[LDSF];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = W1X4 ? 0 : wave >> 1, wn = W1X4 ? wave : wave & 1;
  const int l32 = lane & 31, hl = lane >> 5;
  const int rin = lane >> 2, chunk = (lane & 3) ^ ((rin >> 2) & 3);
  // first of the 16 A rows that load i of this wave fills
  auto a_row0 = [&](int i) { return W1X4 ? 16 * (wave & 1) : 16 * (4 * i + wave); };
  const float* ag[NA];
  const float* bg[W2N / 64];
  // implicit conv (A_CONV): per row, the top-left input coordinate of its
  // window and the address of that (possibly padded) pixel's channel
  // 4 * chunk; a K step of 16 channels lies inside one tap (Cin % 16 == 0),
  // so a lane's 16 bytes are contiguous. Taps outside the image, and rows
  // past M, load from g_zero16.
  int ohs[NA], ows[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int mr = m0 + a_row0(i) + rin;
    const int64_t m = min(mr, M - 1);
    if constexpr (CONV) {
      const int hw = p.cHo * p.cWo;
      const int img = (int)(m / hw), rem = (int)(m - (int64_t)img * hw);
      const int oh = rem / p.cWo, ow = rem - oh * p.cWo;
      const int ih0 = oh * p.cs - p.cp;
      ows[i] = ow * p.cs - p.cp;
      ag[i] = p.A + (((int64_t)img * p.cH + ih0) * p.cW + ows[i]) * p.cCin + 4 * chunk;
      ohs[i] = mr < M ? ih0 : -(1 << 20);  // rows past M: never in bounds
    } else {
      ag[i] = p.A + m * p.lda + 4 * chunk;
    }
  }
#pragma unroll
  for (int i = 0; i < W2N / 64; ++i) {
    const int64_t n = min(n0 + 16 * (4 * i + wave) + rin, N - 1);
    bg[i] = p.B + n * p.ldb + 4 * chunk;
  }
  const uint32_t lds0 = lds_addr(lds);
  // conv tap state of the next step to issue (wave-uniform)
  int tkh = 0, tkw = 0, tic = 0;
  const float* zrow = g_zero16 + 4 * chunk;
#define GS_F2_ISSUE(BUF, K0)                                                                 \
  {                                                                                          \
    if constexpr (CONV) {                                                                    \
      const int64_t toff = ((int64_t)tkh * p.cW + tkw) * p.cCin + tic;                       \
      _Pragma("unroll") for (int i = 0; i < NA; ++i) {                                       \
        const bool ok = (unsigned)(ohs[i] + tkh) < (unsigned)p.cH &&                          \
                        (unsigned)(ows[i] + tkw) < (unsigned)p.cW;                            \
        lds_dma16(ok ? ag[i] + toff : zrow, lds0 + ((BUF) * FSTAGE + a_row0(i) * FK) * 4);   \
      }                                                                                      \
      tic += FK;                                                                             \
      if (tic == p.cCin) {                                                                   \
        tic = 0;                                                                             \
        if (++tkw == p.ckw) {                                                                 \
          tkw = 0;                                                                           \
          ++tkh;                                                                             \
        }                                                                                    \
      }                                                                                      \
    } else {                                                                                 \
      _Pragma("unroll") for (int i = 0; i < NA; ++i)                                         \
        lds_dma16(ag[i] + (K0), lds0 + ((BUF) * FSTAGE + a_row0(i) * FK) * 4);               \
    }                                                                                        \
    _Pragma("unroll") for (int i = 0; i < W2N / 64; ++i)                                     \
      lds_dma16(bg[i] + (K0), lds0 + ((BUF) * FSTAGE + (BM + 16 * (4 * i + wave)) * FK) * 4); \
  }
  const int swz = (l32 >> 2) & 3;
  const int ra0 = (wm * 32 * WTM + l32) * FK, rb0 = (wn * (W1X4 ? 32 : 64) + l32) * FK;
  floatx16 c00 = {}, c01 = {}, c10 = {}, c11 = {}, c20 = {}, c21 = {}, c30 = {}, c31 = {};
  // K range: all of K, or (32-row form, split launch) range blockIdx.y of
  // batch.ksplit in 32-deep steps (every range non-empty, checked on the host)
  int kbeg = 0, kend = K;
  if constexpr (W1X4)
    if (batch.ksplit > 1) split_range(K, batch.ksplit, BK, kbeg, kend);
  int buf = 0;
  GS_F2_ISSUE(0, kbeg)
  for (int k0 = kbeg; k0 < kend; k0 += FK) {
    // each wave waits for its own NA + 2 loads of step k0
    if (k0 + FK < kend) {
      GS_F2_ISSUE(buf ^ 1, k0 + FK)
      if constexpr (BM == 256)
        asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
      else if constexpr (BM == 192)
        asm volatile("s_waitcnt vmcnt(5)\n\ts_barrier" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(3)\n\ts_barrier" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    }
    const float* as = lds + buf * FSTAGE;
    const float* bs = as + BM * FK;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int co = ((2 * hl + u) ^ swz) << 2;
      const fx4 a0 = *(const fx4*)(as + ra0 + co);
      fx4 a1 = {}, a2 = {}, a3 = {};
      if constexpr (WTM >= 2) a1 = *(const fx4*)(as + ra0 + 32 * FK + co);
      if constexpr (WTM >= 3) a2 = *(const fx4*)(as + ra0 + 64 * FK + co);
      if constexpr (WTM == 4) a3 = *(const fx4*)(as + ra0 + 96 * FK + co);
      const fx4 b0 = *(const fx4*)(bs + rb0 + co);
      fx4 b1 = {};
      if constexpr (!W1X4) b1 = *(const fx4*)(bs + rb0 + 32 * FK + co);
#define GS_F2_MM(X)                                                                          \
  c00 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.X, b0.X, c00, 0, 0, 0);                      \
  if constexpr (!W1X4) c01 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.X, b1.X, c01, 0, 0, 0); \
  if constexpr (WTM >= 2) {                                                                  \
    c10 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.X, b0.X, c10, 0, 0, 0);                    \
    c11 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.X, b1.X, c11, 0, 0, 0);                    \
  }                                                                                          \
  if constexpr (WTM >= 3) {                                                                  \
    c20 = __builtin_amdgcn_mfma_f32_32x32x2f32(a2.X, b0.X, c20, 0, 0, 0);                    \
    c21 = __builtin_amdgcn_mfma_f32_32x32x2f32(a2.X, b1.X, c21, 0, 0, 0);                    \
  }                                                                                          \
  if constexpr (WTM == 4) {                                                                  \
    c30 = __builtin_amdgcn_mfma_f32_32x32x2f32(a3.X, b0.X, c30, 0, 0, 0);                    \
    c31 = __builtin_amdgcn_mfma_f32_32x32x2f32(a3.X, b1.X, c31, 0, 0, 0);                    \
  }
      GS_F2_MM(x)
      GS_F2_MM(y)
      GS_F2_MM(z)
      GS_F2_MM(w)
#undef GS_F2_MM
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    buf ^= 1;
  }
#undef GS_F2_ISSUE
  const int mw = m0 + wm * 32 * WTM, nw = n0 + wn * (W1X4 ? 32 : 64);
  float* stage = lds + wave * 32 * (W1X4 ? W2_SS1 : W2_SS);
  if constexpr (W1X4) {
    if (batch.ksplit > 1) {
      // raw partial of this K range: part[blockIdx.y][row][col] (half-waves
      // store 128 contiguous bytes of one row); gemm_splitk_reduce sums the
      // ranges and applies the epilogue
      float* part = p.part + (int64_t)blockIdx.y * M * N;
      const int col = nw + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = mw + 8 * (r >> 2) + 4 * hl + (r & 3);
        if (row < M && col < N) part[(int64_t)row * N + col] = c00[r];
      }
    } else if (p.flags & EPI_ROPE) {
      w2_epi_row<true, 1>(p, c00, c00, mw, nw, stage, lane, l32, hl);
    } else {
      w2_epi_row<false, 1>(p, c00, c00, mw, nw, stage, lane, l32, hl);
    }
  } else if (p.flags & EPI_ROPE) {
    w2_epi_row<true>(p, c00, c01, mw, nw, stage, lane, l32, hl);
    if constexpr (WTM >= 2) w2_epi_row<true>(p, c10, c11, mw + 32, nw, stage, lane, l32, hl);
    if constexpr (WTM >= 3) w2_epi_row<true>(p, c20, c21, mw + 64, nw, stage, lane, l32, hl);
    if constexpr (WTM == 4) w2_epi_row<true>(p, c30, c31, mw + 96, nw, stage, lane, l32, hl);
  } else {
    w2_epi_row<false>(p, c00, c01, mw, nw, stage, lane, l32, hl);
    if constexpr (WTM >= 2) w2_epi_row<false>(p, c10, c11, mw + 32, nw, stage, lane, l32, hl);
    if constexpr (WTM >= 3) w2_epi_row<false>(p, c20, c21, mw + 64, nw, stage, lane, l32, hl);
    if constexpr (WTM == 4) w2_epi_row<false>(p, c30, c31, mw + 96, nw, stage, lane, l32, hl);
  }
}

template <int ALOAD, bool A_RELU, bool BSPLIT>
__global__ __launch_bounds__(256, 2) void gemm_x6_kernel(GemmBatch batch) {
  constexpr int BLAYOUT = B_NT;
  const GemmArgs& p = batch.g[blockIdx.z];
  const int M = p.M, N = p.N, K = p.K;
  int m0, n0;
  if (!gemm_tile(p, m0, n0)) return;

  // unpadded rows of 32 bf16 (four 16-byte chunks), chunk c of row r at slot
  // c ^ ((r >> 2) & 3): the MFMA reads of 16 consecutive rows at one chunk
  // and the split writes of 4 consecutive rows hit distinct bank groups
  __shared__ __attribute__((aligned(16))) __bf16 As[3][BM][BK];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[3][BN][BK];
#define GS_X6_SW(R, K) ((((K) >> 3) ^ (((R) >> 2) & 3)) << 3 | ((K) & 7))

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, hl = lane >> 5;
  const int lrow = tid >> 3, lc4 = (tid & 7) * 4;

  GS_ROW_STATE()
  int boff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = n0 + lrow + 32 * i;
    boff[i] = min(n, N - 1) * (int)p.ldb + lc4;
  }
  const int bncol = 0;  // NN-layout state of the shared loader macro (unused here)
  // pre-split B: rows tid/4 + 64*j (j < 2), 8 bf16 at column 8*(tid%4) per plane
  const __bf16* Bh = (const __bf16*)p.Bh;
  const int brow = tid >> 2, bc8 = (tid & 3) * 8;
  int bo[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + brow + 64 * j;
    bo[j] = min(n, N - 1) * (int)p.ldb + bc8;
  }
  // two register stages: the loads of K step k + 2 are issued at step k, so
  // they have two steps of MFMA work to land (one step of this kernel is a
  // third of the fp32 kernel's MFMA time, too short to hide them alone)
  fx4 ra0[4] = {}, ra1[4] = {}, rb0[BSPLIT ? 1 : 4], rb1[BSPLIT ? 1 : 4], lgb0[2] = {},
      lgb1[2] = {};
  bool aok0[4] = {}, aok1[4] = {};
  // A of the next step, fixed up and split into its three planes during this
  // step's MFMAs (so only the LDS stores remain between the barriers)
  bf16x4 sah[4], sam[4], sal[4];
  bf16x8 rbp0[BSPLIT ? 3 : 1][2], rbp1[BSPLIT ? 3 : 1][2];
  const fx4 zero4 = mk4(0.f, 0.f, 0.f, 0.f);
  floatx16 acc00 = {}, acc01 = {}, acc10 = {}, acc11 = {};
  // loads of one K step into register stage S (0 or 1), through the shared
  // loader macros (which write ra / rb)
#define GS_X6_LOAD(K0, S)                                                        \
  {                                                                              \
    fx4* const ra = S ? ra1 : ra0;                                               \
    fx4* const rb = S ? rb1 : rb0;                                               \
    fx4* const lgb = S ? lgb1 : lgb0;                                            \
    bool* const aok = S ? aok1 : aok0;                                           \
    (void)rb;                                                                    \
    (void)lgb;                                                                   \
    (void)aok;                                                                   \
    GS_LOAD_A(K0)                                                                \
    if (BSPLIT) {                                                                \
      bf16x8(*const rbp)[2] = S ? rbp1 : rbp0;                                   \
      _Pragma("unroll") for (int t = 0; t < 3; ++t)                              \
      _Pragma("unroll") for (int j = 0; j < 2; ++j) {                            \
        const bf16x8 w = *(const bf16x8*)(Bh + t * p.bh_plane + bo[j] + (K0));   \
        rbp[t][j] = w;                                                           \
      }                                                                          \
    } else {                                                                     \
      GS_LOAD_B_F32(K0)                                                          \
    }                                                                            \
  }
  // fix-up and split of the A values in register stage S into sah/sam/sal
#define GS_X6_PREP(S)                                                            \
  {                                                                              \
    fx4* const ra = S ? ra1 : ra0;                                               \
    fx4* const lgb = S ? lgb1 : lgb0;                                            \
    bool* const aok = S ? aok1 : aok0;                                           \
    (void)lgb;                                                                   \
    (void)aok;                                                                   \
    GS_FIX_A()                                                                   \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) split3(ra[i], sah[i], sam[i], sal[i]); \
  }
  // one K step: the A planes split during the previous step and B's planes
  // from register stage S into LDS, then the loads of step k0 + 2 BK into the
  // freed stage, then the MFMAs with the split of step k0 + BK beside them
#define GS_X6_STEP(S)                                                            \
  {                                                                              \
    fx4* const rb = S ? rb1 : rb0;                                               \
    __syncthreads();                                                             \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                              \
      const int sa_ = GS_X6_SW(lrow + 32 * i, lc4);                              \
      *(bf16x4*)&As[0][lrow + 32 * i][sa_] = sah[i];                             \
      *(bf16x4*)&As[1][lrow + 32 * i][sa_] = sam[i];                             \
      *(bf16x4*)&As[2][lrow + 32 * i][sa_] = sal[i];                             \
      if (!BSPLIT) {                                                             \
        bf16x4 h, m, l;                                                          \
        split3(rb[i], h, m, l);                                                  \
        *(bf16x4*)&Bs[0][lrow + 32 * i][sa_] = h;                                \
        *(bf16x4*)&Bs[1][lrow + 32 * i][sa_] = m;                                \
        *(bf16x4*)&Bs[2][lrow + 32 * i][sa_] = l;                                \
      }                                                                          \
    }                                                                            \
    if (BSPLIT) {                                                                \
      bf16x8(*const rbp)[2] = S ? rbp1 : rbp0;                                   \
      _Pragma("unroll") for (int t = 0; t < 3; ++t)                              \
      _Pragma("unroll") for (int j = 0; j < 2; ++j)                              \
        *(bf16x8*)&Bs[t][brow + 64 * j][GS_X6_SW(brow + 64 * j, bc8)] = rbp[t][j]; \
    }                                                                            \
    __syncthreads();                                                             \
    if (k0 + 2 * BK < kend) GS_X6_LOAD(k0 + 2 * BK, S)                           \
    GS_X6_PREP(1 - S)                                                            \
    GS_X6_MMA()                                                                  \
    k0 += BK;                                                                    \
  }
#define GS_X6_MMA()                                                              \
  _Pragma("unroll") for (int sl = 0; sl < 2; ++sl) {                             \
    const int kc = GS_X6_SW(l32, sl * 16 + hl * 8); /* rows wm*64 + l32 (+32) */ \
    bf16x8 a0[3], a1[3], b0[3], b1[3];                                           \
    _Pragma("unroll") for (int t = 0; t < 3; ++t) {                              \
      a0[t] = *(const bf16x8*)&As[t][wm * 64 + l32][kc];                         \
      a1[t] = *(const bf16x8*)&As[t][wm * 64 + 32 + l32][kc];                    \
      b0[t] = *(const bf16x8*)&Bs[t][wn * 64 + l32][kc];                         \
      b1[t] = *(const bf16x8*)&Bs[t][wn * 64 + 32 + l32][kc];                    \
    }                                                                            \
    GS_X6(2, 0)                                                                  \
    GS_X6(0, 2)                                                                  \
    GS_X6(1, 1)                                                                  \
    GS_X6(1, 0)                                                                  \
    GS_X6(0, 1)                                                                  \
    GS_X6(0, 0)                                                                  \
  }
#define GS_X6(TA, TB)                                                                \
  acc00 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[TA], b0[TB], acc00, 0, 0, 0);   \
  acc01 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[TA], b1[TB], acc01, 0, 0, 0);   \
  acc10 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[TA], b0[TB], acc10, 0, 0, 0);   \
  acc11 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[TA], b1[TB], acc11, 0, 0, 0);

  int kbeg, kend;
  split_range(K, batch.ksplit, BK, kbeg, kend);
  int k0 = kbeg;
  GS_X6_LOAD(kbeg, 0)
  if (kbeg + BK < kend) GS_X6_LOAD(kbeg + BK, 1)
  GS_X6_PREP(0)
  while (true) {
    GS_X6_STEP(0)
    if (k0 >= kend) break;
    GS_X6_STEP(1)
    if (k0 >= kend) break;
  }
#undef GS_X6
#undef GS_X6_MMA
#undef GS_X6_STEP
#undef GS_X6_PREP
#undef GS_X6_LOAD
#undef GS_X6_SW
  if (batch.ksplit > 1)
    store_partial(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
  else
    gemm_epilogue(p, acc00, acc01, acc10, acc11, m0, n0, wm, wn, l32, hl);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

// The staged epilogue of the one-wave-per-SIMD kernels stores 4 columns per
// lane with vector accesses.
bool row_epi_ok(const GemmArgs& g) {
  if (g.flags & EPI_SCATTER)  // 4-column segments stay within one output pixel
    return g.sc_C % 4 == 0 && g.sc_Cout % 4 == 0 && g.N % 4 == 0 && aligned16(g.C) &&
           !(g.flags & (EPI_RES1 | EPI_RES2 | EPI_ROPE | EPI_DUAL));
  if (g.N % 4 || g.ldc % 4 || !aligned16(g.C)) return false;
  if ((g.flags & EPI_RES1) && (g.ldr1 % 4 || !aligned16(g.R1))) return false;
  if ((g.flags & EPI_RES2) && (g.ldr2 % 4 || !aligned16(g.R2))) return false;
  if ((g.flags & EPI_DUAL) && !aligned16(g.C2)) return false;
  return true;
}

std::string gemm_prof_name(const char* base, const GemmBatch& b) {
  std::string n = base;
  if (prof_per_shape()) {
    const GemmArgs& g = b.g[0];
    n += " M=" + std::to_string(g.M) + " N=" + std::to_string(g.N) + " K=" + std::to_string(g.K) +
         " groups=" + std::to_string(b.ngroups);
    if (g.flags & EPI_GELU) n += " gelu";
    if (b.ksplit > 1) n += " splitk=" + std::to_string(b.ksplit);
    if (b.tphase_q) n += " per-round";
  }
  return n;
}

}  // namespace

int check_gemm(const GemmArgs& a, int aload, int blayout, bool bf16) {
  GS_REQUIRE(a.M >= 0 && a.N > 0 && a.K > 0, "gemm: bad sizes");
  GS_REQUIRE(a.K % BK == 0, "gemm: K must be a multiple of 32");
  GS_REQUIRE(a.A && a.B && a.C, "gemm: null operand");
  GS_REQUIRE(aligned16(a.A) && aligned16(a.B), "gemm: operands must be 16-byte aligned");
  GS_REQUIRE(a.ldb % 4 == 0, "gemm: ldb must be a multiple of 4");
  if (aload != A_CONV && aload != A_CONV_H)
    GS_REQUIRE(a.lda % 4 == 0 && a.lda >= (aload == A_CONCAT ? a.K1 : a.K), "gemm: bad lda");
  if (aload == A_LN)
    GS_REQUIRE(!bf16 && a.ln_stats && a.ln_g && a.ln_b && aligned16(a.ln_g) && aligned16(a.ln_b),
               "gemm: the fused LayerNorm load needs row statistics, gamma and beta "
               "(fp32 kernels)");
  if (aload == A_PLAIN_H || aload == A_CONV_H)
    GS_REQUIRE(blayout == B_NT && bf16, "gemm: bf16 A needs the bf16 kernel and the NT layout");
  if (aload == A_CONCAT)
    GS_REQUIRE(a.A2 && aligned16(a.A2) && a.K1 % BK == 0 && a.K1 > 0 && a.K1 < a.K &&
                   a.lda2 % 4 == 0 && a.lda2 >= a.K - a.K1,
               "gemm: bad concat operand");
  if (aload == A_CONV || aload == A_CONV_H) {
    GS_REQUIRE(a.cCin % BK == 0, "conv: Cin must be a multiple of 32");
    GS_REQUIRE(a.ck > 0 && a.ckw > 0 && a.cs > 0 && a.cp >= 0, "conv: bad kernel geometry");
    GS_REQUIRE(a.K == a.ck * a.ckw * a.cCin, "conv: K != kh*kw*Cin");
    GS_REQUIRE(a.cHo == (a.cH + 2 * a.cp - a.ck) / a.cs + 1 &&
                   a.cWo == (a.cW + 2 * a.cp - a.ckw) / a.cs + 1,
               "conv: output grid mismatch");
    GS_REQUIRE(a.M % (a.cHo * a.cWo) == 0, "conv: M must be images*Ho*Wo");
  }
  if (blayout == B_NT)
    GS_REQUIRE(a.ldb >= a.K && (int64_t)a.N * a.ldb < ((int64_t)1 << 31), "gemm: bad ldb");
  else GS_REQUIRE(a.N % 4 == 0 && a.ldb >= a.N, "gemm: NN layout needs N % 4 == 0");
  if (a.flags & EPI_BIAS) GS_REQUIRE(a.bias != nullptr, "gemm: null bias");
  if (a.flags & EPI_RES1) GS_REQUIRE(a.R1 != nullptr, "gemm: null residual");
  if (a.flags & EPI_RES2) GS_REQUIRE(a.R2 != nullptr, "gemm: null residual 2");
  if (a.flags & EPI_ROPE)
    GS_REQUIRE(a.rope_cos && a.rope_sin && a.rope_ncols % 64 == 0 &&
                   a.rope_ncols <= a.N && a.tok_per_img > 0 && a.grid_w > 0,
               "gemm: bad rope epilogue");
  if (a.flags & EPI_DUAL)
    GS_REQUIRE(a.C2 != nullptr && !(a.flags & EPI_SCATTER), "gemm: bad dual store");
  if (a.flags & EPI_DUAL_RELU_H)
    GS_REQUIRE(a.flags & EPI_DUAL, "gemm: the ReLU'd bf16 copy is a form of the dual store");
  if (a.flags & EPI_ROPE)
    GS_REQUIRE(!(a.flags & (EPI_RES1 | EPI_RES2)) && a.M < (1 << 22) && a.tok_per_img > 0 &&
                   a.grid_w > 0,
               "gemm: RoPE excludes residual epilogues and needs M < 2^22");
  if (a.flags & EPI_BF16OUT)
    GS_REQUIRE(!(a.flags & EPI_DUAL) && ((a.flags & EPI_SCATTER) || a.ldc % 4 == 0),
               "gemm: bf16 output excludes dual stores");
  if (a.flags & EPI_LNOUT)
    GS_REQUIRE(!(a.flags & ~(EPI_BIAS | EPI_RES1 | EPI_RES2 | EPI_LNOUT)) && a.N % 4 == 0 &&
                   a.N <= 4096 && a.ldc == a.N && a.lnout && a.lnout_g && a.lnout_b &&
                   aligned16(a.lnout) && aligned16(a.lnout_g) && aligned16(a.lnout_b) &&
                   aligned16(a.C) && (!(a.flags & EPI_BIAS) || aligned16(a.bias)) &&
                   (!(a.flags & EPI_RES1) || (a.ldr1 % 4 == 0 && aligned16(a.R1))) &&
                   (!(a.flags & EPI_RES2) || (a.ldr2 % 4 == 0 && aligned16(a.R2))),
               "gemm: the LayerNorm output takes bias / residual epilogues, N % 4 == 0, "
               "N <= 4096, ldc == N and 16-byte aligned operands");
  if (a.flags & EPI_SCATTER)
    GS_REQUIRE(a.sc_r > 0 && a.sc_C > 0 && a.N == a.sc_r * a.sc_r * a.sc_C &&
                   a.sc_Cout <= a.sc_C && a.sc_gh > 0 && a.sc_gw > 0 &&
                   a.M % (a.sc_gh * a.sc_gw) == 0,
               "gemm: bad scatter epilogue");
  else
    GS_REQUIRE(a.ldc >= a.N, "gemm: ldc < N");
  return 0;
}

namespace {

// Split factor for a launch that would leave CUs idle: the smallest divisor S
// of the K-step count (at least 4 K steps per range, S <= 16) that gives
// kSplitTarget workgroups, else the largest such divisor; 1 when the launch
// already has that many tiles, when there is no scratch, or for scatter
// epilogues. kSplitTarget (~1.7 workgroups per CU) is measured: over the
// one-image / one-pair encoder and decoder shapes (M 768..1536, N 768..4096,
// K 768..4096) the fastest split was the smallest giving >= 432 workgroups.
constexpr int kSplitTarget = 432;
constexpr int kNumCUs = 256;  // MI355X compute units
bool splitk_eligible(const GemmBatch& b) {
  if (!b.part_ws || !aligned16(b.part_ws)) return false;
  const GemmArgs& g0 = b.g[0];
  for (int i = 0; i < b.ngroups; ++i) {
    const GemmArgs& g = b.g[i];
    if (g.M != g0.M || g.N != g0.N || g.K != g0.K) return false;
    if ((g.flags & EPI_SCATTER) || g.N % 4 || g.ldc % 4 || !aligned16(g.C)) return false;
    if ((g.flags & EPI_BIAS) && !aligned16(g.bias)) return false;
    if ((g.flags & EPI_RES1) && (g.ldr1 % 4 || !aligned16(g.R1))) return false;
    if ((g.flags & EPI_RES2) && (g.ldr2 % 4 || !aligned16(g.R2))) return false;
    if ((g.flags & EPI_DUAL) && !aligned16(g.C2)) return false;
  }
  return true;
}

int plan_ksplit(const GemmBatch& b, int max_tiles) {
  if (!splitk_eligible(b)) return 1;
  const GemmArgs& g0 = b.g[0];
  const int tiles = max_tiles * b.ngroups;
  if (tiles >= kSplitTarget) return 1;
  const int steps = g0.K / BK;
  int best = 1;
  for (int cand = 2; cand <= 16; ++cand) {
    if (steps % cand || steps / cand < 4) continue;
    if ((int64_t)cand * g0.M * g0.N * b.ngroups > b.part_ws_elems) continue;
    best = cand;
    if (tiles * cand >= kSplitTarget) break;
  }
  return best;
}

// Split factor of a direct-to-LDS launch with fewer tiles than one round of
// the 256 x 128 kernel. That kernel keeps the matrix cores busy at one
// workgroup per CU (its double buffer hides the loads), so a CU's time is its
// workgroup count times the K steps of each, and a split costs its partial
// tiles' round trip through the scratch. Cost in units of one workgroup K
// step (1.88 us), fitted to 95 timed launches of the one-image / one-pair
// encoder and decoder shapes (M 768..1536, N 768..4096, K 768..4096, S 1..16):
//   ceil(S * tiles / CUs) * ceil(steps / S) + [S > 1] (0.627 S M N g / 1e6 - 6.1)
// The S it minimises is the fastest measured one on 13 of the 14 shapes and
// within 2 % on the last; the 432-workgroup rule of plan_ksplit was up to
// 22 % slower on six of them. Ranges keep at least 4 K steps.
int plan_ksplit_dl(const GemmBatch& b, int max_tiles) {
  if (!splitk_eligible(b)) return 1;
  const GemmArgs& g0 = b.g[0];
  const int tiles = max_tiles * b.ngroups, steps = g0.K / BK;
  const double mn = (double)g0.M * g0.N * b.ngroups;
  int best = 1;
  double best_cost = 0.0;
  for (int S = 1; S <= 16; ++S) {
    if (S > 1 && (steps / S < 4 || (int64_t)S * g0.M * g0.N * b.ngroups > b.part_ws_elems))
      break;
    const double per_cu = (double)((tiles * S + kNumCUs - 1) / kNumCUs);
    const double cost = per_cu * ((steps + S - 1) / S) + (S > 1 ? 0.627 * S * mn / 1e6 - 6.1 : 0.0);
    if (S == 1 || cost < best_cost) {
      best = S;
      best_cost = cost;
    }
  }
  return best;
}

// The split-K reduce pass of a launch (with the row LayerNorm for EPI_LNOUT).
void launch_reduce(const GemmBatch& b, dim3 rgrid, hipStream_t s) {
  if (b.g[0].flags & EPI_LNOUT) {
    const dim3 g((unsigned)((b.g[0].M + 3) / 4), b.ngroups);
    if (b.g[0].N <= 1024)
      hipLaunchKernelGGL(gemm_splitk_reduce_ln<4>, g, dim3(256), 0, s, b);
    else
      hipLaunchKernelGGL(gemm_splitk_reduce_ln<16>, g, dim3(256), 0, s, b);
  } else {
    hipLaunchKernelGGL(gemm_splitk_reduce, rgrid, dim3(256), 0, s, b);
  }
}

// EPI_LNOUT of an unsplit launch: the LayerNorm kernel over the finished C.
int post_layernorm(const GemmBatch& b, hipStream_t s) {
  if (b.ksplit > 1 || !(b.g[0].flags & EPI_LNOUT)) return 0;
  LnBatch lb;
  lb.ngroups = b.ngroups;
  for (int i = 0; i < b.ngroups; ++i) {
    const GemmArgs& g = b.g[i];
    lb.g[i] = LnArgs{g.C, g.lnout_g, g.lnout_b, g.lnout, g.M, g.N, g.lnout_eps};
  }
  return launch_layernorm(lb, s);
}

}  // namespace

int launch_gemm(const GemmBatch& b_in, int aload, int blayout, bool a_relu,
                hipStream_t s, bool bf16) {
  GS_REQUIRE(b_in.ngroups >= 1 && b_in.ngroups <= kMaxGroups, "gemm: bad group count");
  GemmBatch b = b_in;
  int max_tiles = 0;
  for (int i = 0; i < b.ngroups; ++i) {
    int rc = check_gemm(b.g[i], aload, blayout, bf16);
    if (rc) return rc;
    if (bf16)
      GS_REQUIRE(blayout == B_NT && b.g[i].Bh && aligned16(b.g[i].Bh) && b.g[i].ldb % 8 == 0,
                 "gemm: bf16 needs a 16-byte aligned bf16 weight copy in the NT layout");
    const int t = ((b.g[i].M + BM - 1) / BM) * ((b.g[i].N + BN - 1) / BN);
    max_tiles = t > max_tiles ? t : max_tiles;
  }
  for (int i = 1; i < b.ngroups; ++i)
    GS_REQUIRE((b.g[i].flags & EPI_LNOUT) == (b.g[0].flags & EPI_LNOUT) &&
                   (!(b.g[0].flags & EPI_LNOUT) || b.g[i].M == b.g[0].M),
               "gemm: the LayerNorm output needs the same setting and M in every group");
  if (max_tiles == 0) return 0;
  // fp32 plain / concat rows with NT weights below one round of 256 x 128
  // tiles take the direct-to-LDS kernel, split by its own cost model
  // (measured at one image / one pair: faster than the register-staged
  // kernel at every split factor of those shapes)
  const bool dl_ok = !bf16 && blayout == B_NT && !a_relu && (aload == A_PLAIN || aload == A_CONCAT);
  const bool dl_small = dl_ok && (b.kernel == 2 || (b.kernel == 0 && max_tiles * b.ngroups < kF2MinTiles));
  // small launches whose 64 x 128 tiles give every CU at least one: the
  // 64-row form of the direct-to-LDS kernel, unsplit (no reduce pass); plain
  // rows, and implicit convs without a ReLU prologue below one round of the
  // 192-row form
  int t64 = 0, tot64 = 0;
  const bool conv64 = !bf16 && aload == A_CONV && !a_relu && blayout == B_NT;
  bool w64 = ((dl_small && aload == A_PLAIN) || conv64) && b.kernel == 0 && b.ksplit == 0;
  int tot192c = 0;
  for (int i = 0; w64 && i < b.ngroups; ++i) {
    const GemmArgs& g = b.g[i];
    const int t = ((g.M + 63) / 64) * ((g.N + W2N - 1) / W2N);
    t64 = std::max(t64, t);
    tot64 += t;
    tot192c += ((g.M + 191) / 192) * ((g.N + W2N - 1) / W2N);
    w64 = g.K % 16 == 0 && (conv64 ? g.cCin % 16 == 0 : g.lda % 4 == 0) && aligned16(g.A) &&
          g.ldb % 4 == 0 && aligned16(g.B) && row_epi_ok(g) &&
          (!(g.flags & EPI_ROPE) || g.rope_ncols % 64 == 0);
  }
  w64 = w64 && tot64 >= kW64MinTiles && !(conv64 && tot192c >= kF2MinTiles);
  // the 32-row form, unsplit: smaller plain-row launches whose 32 x 128 tiles
  // still fill the CUs; launches of the 64-row form whose busiest CU would
  // carry more work than the 32-row form's (a 64-row tile is two 32-row
  // tiles of work; at most six 32-row tiles per CU, one round at up to eight
  // workgroups per CU); and, below both, launches whose busiest CU carries
  // no more work than under the split 128 x 128 kernel
  int t32 = 0, tot32 = 0;
  bool w32 = dl_small && aload == A_PLAIN && b.kernel == 0 && b.ksplit == 0;
  for (int i = 0; w32 && i < b.ngroups; ++i) {
    const GemmArgs& g = b.g[i];
    const int t = ((g.M + 31) / 32) * ((g.N + W2N - 1) / W2N);
    t32 = std::max(t32, t);
    tot32 += t;
    w32 = g.K % 16 == 0 && g.lda % 4 == 0 && aligned16(g.A) && g.ldb % 4 == 0 &&
          aligned16(g.B) && row_epi_ok(g) && (!(g.flags & EPI_ROPE) || g.rope_ncols % 64 == 0);
  }
  if (w32) {
    const int per_cu32 = (tot32 + kNumCUs - 1) / kNumCUs, per_cu64 = (tot64 + kNumCUs - 1) / kNumCUs;
    if (w64) {
      w32 = tot32 <= 6 * kNumCUs && per_cu32 < 2 * per_cu64;
    } else if (tot32 < kW32MinTiles && (b.g[0].flags & EPI_LNOUT)) {
      // a split launch writes the next LayerNorm in its reduce pass; unsplit,
      // it would take a LayerNorm pass of its own
      w32 = false;
    } else if (tot32 < kW32MinTiles) {
      // against the split 128 x 128 kernel: the busiest CU's multiply-adds
      // at the split its planner picks, ties to the 32-row form (no reduce
      // pass)
      const int S = plan_ksplit_dl(b, max_tiles), steps = b.g[0].K / BK;
      const double work_dl = (double)((max_tiles * b.ngroups * S + kNumCUs - 1) / kNumCUs) *
                             BM * BN * (double)((steps + S - 1) / S) * BK;
      const double work32 = (double)per_cu32 * 32 * W2N * b.g[0].K;
      w32 = work32 <= work_dl;
    }
  }
  // 512-767 tiles of 32 rows that write no LayerNorm (one image's qkv: 576,
  // 2.25 per CU): the 32-row form split in K, as many 32-deep ranges as keep
  // one round at up to eight workgroups per CU
  int s32 = 1;
  if (!w32 && !w64 && tot32 >= 512 && tot32 < kW32MinTiles && !(b.g[0].flags & EPI_LNOUT) &&
      dl_small && aload == A_PLAIN && b.kernel == 0 && b.ksplit == 0 && splitk_eligible(b)) {
    bool ok = true;
    for (int i = 0; ok && i < b.ngroups; ++i) {
      const GemmArgs& g = b.g[i];
      ok = g.K % BK == 0 && g.lda % 4 == 0 && aligned16(g.A) && g.ldb % 4 == 0 &&
           aligned16(g.B) && row_epi_ok(g) && (!(g.flags & EPI_ROPE) || g.rope_ncols % 64 == 0);
    }
    const int steps = b.g[0].K / BK;
    for (int S = 4; ok && S >= 2; --S)
      if (tot32 * S <= 8 * kNumCUs && steps / S >= 4 &&
          (int64_t)S * b.g[0].M * b.g[0].N * b.ngroups <= b.part_ws_elems) {
        w32 = true;
        s32 = S;
        break;
      }
  }
  // launches that write the next LayerNorm (split either way, the reduce
  // writes it): the 32-row form split in K when its busiest CU carries at
  // most 0.8 of the split 128 x 128 kernel's multiply-adds (one pair's
  // encoder proj: three 512-deep 32-row ranges per CU against one 512-deep
  // 128 x 128 range, 1.249 -> 1.103 ms per pair; the one-image proj and fc2,
  // at 0.86 and 0.92 of the work, ran 1-5 % slower split this way)
  if (!w32 && !w64 && tot32 > 0 && (b.g[0].flags & EPI_LNOUT) && dl_small && aload == A_PLAIN &&
      b.kernel == 0 && b.ksplit == 0 && splitk_eligible(b)) {
    bool ok = true;
    for (int i = 0; ok && i < b.ngroups; ++i) {
      const GemmArgs& g = b.g[i];
      ok = g.K % BK == 0 && g.lda % 4 == 0 && aligned16(g.A) && g.ldb % 4 == 0 &&
           aligned16(g.B) && row_epi_ok(g) && (!(g.flags & EPI_ROPE) || g.rope_ncols % 64 == 0);
    }
    const int S = plan_ksplit_dl(b, max_tiles), steps = b.g[0].K / BK;
    const double work_dl = (double)((max_tiles * b.ngroups * S + kNumCUs - 1) / kNumCUs) *
                           BM * BN * (double)((steps + S - 1) / S) * BK;
    double best = 0.0;
    for (int S2 = 2; ok && S2 <= 8; ++S2) {
      if (tot32 * S2 > 8 * kNumCUs || steps / S2 < 4 ||
          (int64_t)S2 * b.g[0].M * b.g[0].N * b.ngroups > b.part_ws_elems)
        break;
      const double w = (double)((tot32 * S2 + kNumCUs - 1) / kNumCUs) * 32 * W2N *
                       (double)((steps + S2 - 1) / S2) * BK;
      if (s32 == 1 || w < best) {
        best = w;
        s32 = S2;
      }
    }
    if (s32 > 1 && best <= 0.8 * work_dl)
      w32 = true;
    else
      s32 = 1;
  }
  if (w32) w64 = false;
  if (w64 || w32) {
    b.ksplit = w32 ? s32 : 1;
  } else if (b.ksplit > 1) {  // requested split
    GS_REQUIRE(splitk_eligible(b), "gemm: this launch cannot split K");
    GS_REQUIRE(b.g[0].K / BK >= b.ksplit &&
                   (int64_t)b.ksplit * b.g[0].M * b.g[0].N * b.ngroups <= b.part_ws_elems,
               "gemm: requested split-K needs a K step per range and must fit the scratch");
  } else {
    b.ksplit = dl_small ? plan_ksplit_dl(b, max_tiles) : plan_ksplit(b, max_tiles);
  }
  int64_t reduce_items = 0;
  if (b.ksplit > 1) {
    GS_REQUIRE(aligned16(b.part_ws), "gemm: split-K scratch must be 16-byte aligned");
    for (int i = 0; i < b.ngroups; ++i) {
      b.g[i].part = b.part_ws + (int64_t)i * b.ksplit * b.g[0].M * b.g[0].N;
      reduce_items = std::max(reduce_items, (int64_t)b.g[i].M * (b.g[i].N / 4));
    }
  }
  dim3 grid(max_tiles, b.ksplit, b.ngroups), block(256);
  const dim3 rgrid((unsigned)((reduce_items + 255) / 256), 1, b.ngroups);
  double flops = 0.0, bytes = 0.0;
  if (prof_on())
    for (int i = 0; i < b.ngroups; ++i) {
      const GemmArgs& g = b.g[i];
      flops += 2.0 * g.M * (double)g.N * g.K;
      const double ea = (aload == A_PLAIN_H || aload == A_CONV_H) ? 2.0 : 4.0, eb = bf16 ? 2.0 : 4.0,
                   ec = (g.flags & EPI_BF16OUT) ? 2.0 : 4.0;
      bytes += ea * g.M * (double)g.K + eb * g.N * (double)g.K + ec * g.M * (double)g.N;
    }
  // bf16 K step: 64 where it divides K and every range keeps a whole step
  int bkc = 2;
  for (int i = 0; i < b.ngroups; ++i)
    if (b.g[i].K % (BK * 2) || b.g[i].K / (BK * 2) < b.ksplit) bkc = 1;
#define GS_GEMM_BF16_CASE(AL, RL)                                             \
  if (bf16 && aload == AL && a_relu == RL) {                                  \
    hipEvent_t ev = prof_start(s);                                            \
    if (bkc == 2)                                                             \
      hipLaunchKernelGGL((gemm_bf16_kernel<AL, RL, 2>), grid, block, 0, s, b); \
    else                                                                      \
      hipLaunchKernelGGL((gemm_bf16_kernel<AL, RL, 1>), grid, block, 0, s, b); \
    if (b.ksplit > 1)                                                         \
      launch_reduce(b, rgrid, s);                                              \
    GS_CHECK_HIP(hipGetLastError());                                          \
    if (ev) prof_stop(s, ev, gemm_prof_name("gemm_bf16_kernel<" #AL "," #RL ">", b).c_str(), \
                      flops, bytes);                                          \
    return post_layernorm(b, s);                                              \
  }
  // large unsplit launches with bf16 activations: the 256 x 128 kernel (at
  // least two of its tiles per CU). Measured at config 4 against the 128 x 128
  // kernel: encoder fc1 873 against 648 TFLOP/s, qkv 742 against 562, fc2 846
  // against 764; a 256 x 256 kernel at one workgroup per CU, which it replaced,
  // ran fc2 at 812 and lost at K <= 1024 (its epilogue is exposed)
  // Implicit convs on a bf16 input (A_CONV_H) take its 192-row form with the
  // per-tap gather (the gather state of 256-row tiles does not fit the
  // three-workgroup register budget).
  if (bf16 && (aload == A_PLAIN_H || aload == A_CONV_H) && !a_relu && b.ksplit == 1) {
    const bool conv = aload == A_CONV_H;
    const int bm = conv ? 192 : 256;
    int wt = 0, wtot = 0, kmin = b.g[0].K;
    bool ok = true;
    for (int i = 0; i < b.ngroups; ++i) {
      const GemmArgs& g = b.g[i];
      kmin = std::min(kmin, g.K);
      const int t = ((g.M + bm - 1) / bm) * ((g.N + W2N - 1) / W2N);
      wt = std::max(wt, t);
      wtot += t;
      ok = ok && g.K % W2K == 0 && (conv ? g.cCin % W2K == 0 : g.lda % 8 == 0) &&
           aligned16(g.A) && g.ldb % 8 == 0 && aligned16(g.Bh) && row_epi_ok(g) &&
           (!(g.flags & EPI_ROPE) || g.rope_ncols % 64 == 0);
    }
    if (ok && wtot >= 512) {
      hipEvent_t ev = prof_start(s);
      if (conv)
        hipLaunchKernelGGL((gemm_bf16_w2_kernel<192, true, 2>), dim3(wt, 1, b.ngroups), dim3(256),
                           0, s, b);
      else if (kmin >= kW2ThreeStageMinK)
        hipLaunchKernelGGL((gemm_bf16_w2_kernel<256, false, 3>), dim3(wt, 1, b.ngroups), dim3(256),
                           0, s, b);
      else
        hipLaunchKernelGGL((gemm_bf16_w2_kernel<256, false, 2>), dim3(wt, 1, b.ngroups), dim3(256),
                           0, s, b);
      GS_CHECK_HIP(hipGetLastError());
      if (ev)
        prof_stop(s, ev,
                  gemm_prof_name(conv ? "gemm_bf16_w2_kernel<192,A_CONV_H>"
                                 : kmin >= kW2ThreeStageMinK ? "gemm_bf16_w2_kernel<A_PLAIN_H,3-stage>"
                                                             : "gemm_bf16_w2_kernel<A_PLAIN_H>",
                                 b).c_str(),
                  flops, bytes);
      return post_layernorm(b, s);
    }
  }
  GS_GEMM_BF16_CASE(A_PLAIN, false)
  GS_GEMM_BF16_CASE(A_PLAIN_H, false)
  GS_GEMM_BF16_CASE(A_CONCAT, false)
  GS_GEMM_BF16_CASE(A_CONV, false)
  GS_GEMM_BF16_CASE(A_CONV, true)
  GS_GEMM_BF16_CASE(A_CONV_H, false)
#undef GS_GEMM_BF16_CASE
  bool presplit = true;
  for (int i = 0; i < b.ngroups; ++i) presplit = presplit && b.g[i].bh_plane > 0;
  if (!bf16 && b.kernel == 3 && presplit)
    for (int i = 0; i < b.ngroups; ++i)
      GS_REQUIRE(b.g[i].Bh && aligned16(b.g[i].Bh) && b.g[i].ldb % 8 == 0 &&
                     b.g[i].bh_plane % 8 == 0,
                 "gemm: pre-split B planes must be 16-byte aligned with ldb % 8 == 0");
#define GS_GEMM_X6_CASE(AL, RL, NM)                                           \
  if (!bf16 && kern == 3 && aload == AL && blayout == B_NT && a_relu == RL) { \
    hipEvent_t ev = prof_start(s);                                            \
    if (presplit)                                                             \
      hipLaunchKernelGGL((gemm_x6_kernel<AL, RL, true>), grid, block, 0, s, b); \
    else                                                                      \
      hipLaunchKernelGGL((gemm_x6_kernel<AL, RL, false>), grid, block, 0, s, b); \
    if (b.ksplit > 1)                                                         \
      launch_reduce(b, rgrid, s);                                              \
    GS_CHECK_HIP(hipGetLastError());                                          \
    if (ev) prof_stop(s, ev, gemm_prof_name("gemm_x6_kernel<" NM ">", b).c_str(), \
                      flops, bytes);                                          \
    return post_layernorm(b, s);                                              \
  }
#define GS_GEMM_CASE(AL, BL, RL)                                              \
  if (!bf16 && aload == AL && blayout == BL && a_relu == RL) {                \
    hipEvent_t ev = prof_start(s);                                            \
    hipLaunchKernelGGL((gemm_f32_kernel<AL, BL, RL>), grid, block, 0, s, b);  \
    if (b.ksplit > 1)                                                         \
      launch_reduce(b, rgrid, s);                                              \
    GS_CHECK_HIP(hipGetLastError());                                          \
    if (ev) prof_stop(s, ev, gemm_prof_name("gemm_f32_kernel<" #AL "," #BL "," #RL ">", b).c_str(), \
                      flops, bytes);                                          \
    return post_layernorm(b, s);                                              \
  }
  // fp32 kernel choice. long-K launches take the direct-to-LDS kernel: its
  // double buffer (64 KB of LDS, two workgroups per CU) pays off from ~2048 K
  // per workgroup, while shorter K (also a long K cut into split ranges) runs
  // faster on the register-staged kernel at three workgroups per CU (measured
  // per shape at config 3 and at one image)
  bool long_k = true;
  for (int i = 0; i < b.ngroups; ++i) long_k = long_k && b.g[i].K / b.ksplit >= 2048;
  int kern = b.kernel;
  if (w32) {
    hipEvent_t ev = prof_start(s);
    hipLaunchKernelGGL((gemm_f32_w2_kernel<32, false>), dim3(t32, b.ksplit, b.ngroups), dim3(256), 0,
                       s, b);
    GS_CHECK_HIP(hipGetLastError());
    if (b.ksplit > 1) {
      launch_reduce(b, rgrid, s);
      GS_CHECK_HIP(hipGetLastError());
    }
    if (ev) prof_stop(s, ev, gemm_prof_name("gemm_f32_w2_kernel<32>", b).c_str(), flops, bytes);
    return post_layernorm(b, s);
  }
  if (w64) {
    hipEvent_t ev = prof_start(s);
    if (conv64)
      hipLaunchKernelGGL((gemm_f32_w2_kernel<64, true>), dim3(t64, 1, b.ngroups), dim3(256), 0, s, b);
    else
      hipLaunchKernelGGL((gemm_f32_w2_kernel<64, false>), dim3(t64, 1, b.ngroups), dim3(256), 0, s, b);
    GS_CHECK_HIP(hipGetLastError());
    if (ev)
      prof_stop(s, ev,
                gemm_prof_name(conv64 ? "gemm_f32_w2_kernel<64,A_CONV>" : "gemm_f32_w2_kernel<64>", b)
                    .c_str(),
                flops, bytes);
    return post_layernorm(b, s);
  }
  if (kern == 0) {
    kern = dl_ok && (long_k || dl_small) ? 2 : 1;
    // large unsplit launches with plain rows or an implicit conv (no ReLU
    // prologue): the 256 x 128 kernel, when its tiles fill the CUs at least
    // once. Convs take its 192-row form: the 256-row form's gather state
    // spills at three workgroups per CU, and measured at the config-3 conv
    // shapes the 192-row form runs 108-130 TFLOP/s against 106-126 for the
    // register-staged conv (the spilling 256-row form 104-122)
    const bool w2_conv = aload == A_CONV;
    if (!bf16 && blayout == B_NT && !a_relu && b.ksplit == 1 && (aload == A_PLAIN || w2_conv)) {
      // 256-row tiles, else 192-row tiles, if they fill the CUs at least once
      int t256 = 0, tot256 = 0, t192 = 0, tot192 = 0;
      bool ok = true;
      for (int i = 0; i < b.ngroups; ++i) {
        const GemmArgs& g = b.g[i];
        const int tn = (g.N + W2N - 1) / W2N;
        const int ta = ((g.M + 255) / 256) * tn, tb = ((g.M + 191) / 192) * tn;
        t256 = std::max(t256, ta);
        tot256 += ta;
        t192 = std::max(t192, tb);
        tot192 += tb;
        ok = ok && g.K % 16 == 0 && (w2_conv ? g.cCin % 16 == 0 : g.lda % 4 == 0) &&
             aligned16(g.A) && g.ldb % 4 == 0 && aligned16(g.B) && row_epi_ok(g) &&
             (!(g.flags & EPI_ROPE) || g.rope_ncols % 64 == 0);
      }
      // the tile height whose tiles fill the last round of workgroup slots
      // best (decoder qkv / kv: 2.25 / 1.5 rounds of 256-row tiles, 3 / 2 of
      // 192-row tiles); ties go to 256 rows
      auto fill = [](int t) {
        const int rounds = (t + kF2MinTiles - 1) / kF2MinTiles;
        return (double)t / ((double)rounds * kF2MinTiles);
      };
      int bm = 0;
      if (ok && tot256 >= kF2MinTiles && !w2_conv) bm = 256;
      if (ok && tot192 >= kF2MinTiles && (bm == 0 || fill(tot192) > fill(tot256))) bm = 192;
      if (bm) {
        bool phased = bm == 256;
        for (int i = 0; i < b.ngroups; ++i) {
          const GemmArgs& g = b.g[i];
          const int t = ((g.M + 255) / 256) * ((g.N + W2N - 1) / W2N);
          phased = phased && g.K >= kF2PhaseMinK && t % 8 == 0 && t > 8 * kF2PhaseTiles;
        }
        if (phased) {
          // one group and one round of tiles per launch (each launch timed on
          // its own, with its share of the group's flops and bytes)
          for (int i = 0; i < b.ngroups; ++i) {
            GemmBatch pb = b;
            pb.g[0] = b.g[i];
            pb.ngroups = 1;
            const GemmArgs& g = b.g[i];
            const int t = ((g.M + 255) / 256) * ((g.N + W2N - 1) / W2N);
            pb.tphase_q = t / 8;
            const double ea = 4.0, ec = (g.flags & EPI_BF16OUT) ? 2.0 : 4.0;
            const double gfl = 2.0 * g.M * (double)g.N * g.K,
                         gby = ea * g.M * (double)g.K + 4.0 * g.N * (double)g.K + ec * g.M * (double)g.N;
            for (int base = 0; base < pb.tphase_q; base += kF2PhaseTiles) {
              pb.tphase_base = base;
              const int per = std::min(kF2PhaseTiles, pb.tphase_q - base);
              hipEvent_t ev = prof_start(s);
              hipLaunchKernelGGL((gemm_f32_w2_kernel<256, false>), dim3(8 * per, 1, 1), dim3(256),
                                 0, s, pb);
              GS_CHECK_HIP(hipGetLastError());
              if (ev)
                prof_stop(s, ev, gemm_prof_name("gemm_f32_w2_kernel<256>", pb).c_str(),
                          gfl * 8 * per / t, gby * 8 * per / t);
            }
          }
          return post_layernorm(b, s);
        }
        hipEvent_t ev = prof_start(s);
        const dim3 grid2(bm == 256 ? t256 : t192, 1, b.ngroups);
        if (bm == 256)
          hipLaunchKernelGGL((gemm_f32_w2_kernel<256, false>), grid2, dim3(256), 0, s, b);
        else if (w2_conv)
          hipLaunchKernelGGL((gemm_f32_w2_kernel<192, true>), grid2, dim3(256), 0, s, b);
        else
          hipLaunchKernelGGL((gemm_f32_w2_kernel<192, false>), grid2, dim3(256), 0, s, b);
        GS_CHECK_HIP(hipGetLastError());
        if (ev) {
          const char* nm = bm == 256 ? "gemm_f32_w2_kernel<256>"
                                     : (w2_conv ? "gemm_f32_w2_kernel<192,A_CONV>"
                                                : "gemm_f32_w2_kernel<192>");
          prof_stop(s, ev, gemm_prof_name(nm, b).c_str(), flops, bytes);
        }
        return post_layernorm(b, s);
      }
    }
  } else {
    GS_REQUIRE(kern >= 1 && kern <= 3 && !bf16, "gemm: unknown fp32 kernel request");
    GS_REQUIRE(kern != 3 || blayout == B_NT, "gemm: the bf16x6 kernel takes NT B");
    GS_REQUIRE(kern != 2 || dl_ok, "gemm: the direct-to-LDS kernel takes plain / concat A, NT B");
  }
#define GS_GEMM_DL_CASE(AL)                                                   \
  if (!bf16 && kern == 2 && aload == AL && blayout == B_NT && !a_relu) {      \
    hipEvent_t ev = prof_start(s);                                            \
    hipLaunchKernelGGL((gemm_f32_dl_kernel<AL>), grid, block, 0, s, b);       \
    if (b.ksplit > 1)                                                         \
      launch_reduce(b, rgrid, s);                                              \
    GS_CHECK_HIP(hipGetLastError());                                          \
    if (ev) prof_stop(s, ev, gemm_prof_name("gemm_f32_dl_kernel<" #AL ">", b).c_str(), \
                      flops, bytes);                                          \
    return post_layernorm(b, s);                                              \
  }
  GS_GEMM_DL_CASE(A_PLAIN)
  GS_GEMM_DL_CASE(A_CONCAT)
#undef GS_GEMM_DL_CASE
  GS_GEMM_X6_CASE(A_PLAIN, false, "A_PLAIN")
  GS_GEMM_X6_CASE(A_LN, false, "A_LN")
  GS_GEMM_X6_CASE(A_CONCAT, false, "A_CONCAT")
  GS_GEMM_X6_CASE(A_CONV, false, "A_CONV")
  GS_GEMM_X6_CASE(A_CONV, true, "A_CONV,relu")
#undef GS_GEMM_X6_CASE
  GS_GEMM_CASE(A_PLAIN, B_NT, false)
  GS_GEMM_CASE(A_LN, B_NT, false)
  GS_GEMM_CASE(A_PLAIN, B_NN, false)
  GS_GEMM_CASE(A_PLAIN, B_NT, true)
  GS_GEMM_CASE(A_CONCAT, B_NT, false)
  GS_GEMM_CASE(A_CONV, B_NT, false)
  GS_GEMM_CASE(A_CONV, B_NT, true)
#undef GS_GEMM_CASE
  set_error("gemm: unsupported loader/layout combination");
  return -1;
}

}  // namespace gs
