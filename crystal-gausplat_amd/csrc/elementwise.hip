// HBM-bound kernels of the path: LayerNorm, patch unfold, bilinear x2
// upsample, RoPE (standalone forms), and the DPT output head split.
#include <math.h>

#include "internal.h"

namespace gs {
namespace {


// LayerNorm#forward_cpu (src/nn/layernorm.cr:192-240): two-pass mean /
// variance, inv_std = 1/sqrt(var + eps), y = (x - mean)*inv_std*gamma + beta.
// One wavefront per row, the row held in registers (D <= 256*NV). The grid
// is capped at the resident workgroups, so each wave steps over rows: gamma
// and beta are loaded once per wave, and the next row's load is in flight
// while the current row is reduced and stored.
constexpr int kLnBlocks = 1280;  // workgroups per group: the 5 per CU that 95 VGPRs leave resident
template <int NV>
__global__ __launch_bounds__(256) void layernorm_kernel(LnBatch bt) {
  const LnArgs& p = bt.g[blockIdx.y];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * 4;
  int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= p.rows) return;
  const int D = p.D, nv = D >> 2;
  const bool out = p.y != nullptr;
  fx4 v[NV], g[NV], bb[NV];
  auto load_row = [&](int64_t r, fx4* dst) {
    const fx4* xr = (const fx4*)(p.x + r * D);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = lane + 64 * i;
      dst[i] = idx < nv ? xr[idx] : mk4(0.f, 0.f, 0.f, 0.f);
    }
  };
  load_row(row, v);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    if (out && idx < nv) {
      g[i] = ((const fx4*)p.gamma)[idx];
      bb[i] = ((const fx4*)p.beta)[idx];
    }
  }
  for (;;) {
    const int64_t next = row + stride;
    fx4 vn[NV];
    if (next < p.rows) load_row(next, vn);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (lane + 64 * i < nv) s += v[i].x + v[i].y + v[i].z + v[i].w;
    const float mean = wave_sum(s) / (float)D;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (lane + 64 * i < nv) {
        const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
        q += a * a + b * b + c * c + d * d;
      }
    }
    const float var = wave_sum(q) / (float)D;
    const float inv = 1.0f / sqrtf(var + p.eps);
    if (p.stats && lane == 0) {  // for GEMMs that apply the normalisation on load
      p.stats[2 * row] = mean;
      p.stats[2 * row + 1] = inv;
    }
    if (out) {
      fx4* yr = (fx4*)(p.y + row * D);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int idx = lane + 64 * i;
        if (idx < nv) {
          fx4 o;
          o.x = (v[i].x - mean) * inv * g[i].x + bb[i].x;
          o.y = (v[i].y - mean) * inv * g[i].y + bb[i].y;
          o.z = (v[i].z - mean) * inv * g[i].z + bb[i].z;
          o.w = (v[i].w - mean) * inv * g[i].w + bb[i].w;
          if (p.y_bf16) {
            typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
            bf16x4_t h;
            h.x = (__bf16)o.x;
            h.y = (__bf16)o.y;
            h.z = (__bf16)o.z;
            h.w = (__bf16)o.w;
            ((bf16x4_t*)((__bf16*)p.y + row * D))[idx] = h;
          } else {
            yr[idx] = o;
          }
        }
      }
    }
    if (next >= p.rows) break;
    row = next;
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = vn[i];
  }
}

// PatchEmbedding#forward unfold (src/nn/vit.cr:56-76): NCHW image -> rows of
// C*p*p in (c, i, j) order. One thread per output fx4.
__global__ void unfold_kernel(const float* __restrict__ img, int32_t B, int32_t H,
                              int32_t W, int32_t p, float* __restrict__ out) {
  const int gw = W / p, gh = H / p;
  const int K = 3 * p * p, K4 = K >> 2;
  const int64_t total = (int64_t)B * gh * gw * K4;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const int64_t m = t / K4;
  const int k = (int)(t - m * K4) * 4;
  const int b = (int)(m / (gh * gw));
  const int rem = (int)(m - (int64_t)b * gh * gw);
  const int ty = rem / gw, tx = rem - ty * gw;
  const int c = k / (p * p), ij = k - c * p * p, i = ij / p, j = ij - i * p;
  const fx4 v = *(const fx4*)(img + (((int64_t)b * 3 + c) * H + ty * p + i) * W +
                                    tx * p + j);
  *(fx4*)(out + m * K + k) = v;
}

// Bilinear x2, align_corners=True (source = dst * (in-1)/(out-1)), NHWC.
// No FMA contraction: a fused sh*oy - y0 moves the lerp weight by an ulp of
// the source coordinate; this kernel is HBM-bound, so it keeps the plain
// operation sequence of the CPU formula.
// One workgroup covers `px` consecutive pixels of one output row, so the
// row's source rows and vertical weights are uniform. Where C / 4 <= 256,
// thread t keeps channel group t % (C / 4) and walks a run of kUpsRun
// consecutive output pixels: neighbouring outputs share source columns (the
// scale is about one half), so the previous pixel's two source columns stay
// in registers and a run of 8 loads about 5 columns instead of 16 (four
// 16-byte loads per 16-byte output held the kernel near half of the HBM
// bandwidth on L1 traffic). Wider rows step over flat element indices.
constexpr int kUpsRun = 8;
// IN_BF16 / OUT_BF16: x / y hold bf16 (element offsets are unchanged).
template <bool IN_BF16, bool OUT_BF16>
__global__ __launch_bounds__(256) void upsample2x_kernel(const float* __restrict__ x,
                                                         int32_t H, int32_t W, int32_t C,
                                                         int32_t blocks_per_row, int32_t px,
                                                         float* __restrict__ y) {
#pragma clang fp contract(off)
  const int Ho = 2 * H, Wo = 2 * W, C4 = C >> 2;
  const int row = (int)(blockIdx.x / (uint32_t)blocks_per_row);  // b * Ho + oy
  const int ox0 = (int)(blockIdx.x - (uint32_t)row * blocks_per_row) * px;
  const int ox1 = min(ox0 + px, Wo);
  const int b = row / Ho;
  const int oy = row - b * Ho;
  const float sh = (float)(H - 1) / (float)(Ho - 1);
  const float sw = (float)(W - 1) / (float)(Wo - 1);
  const float fy = sh * (float)oy;
  const int y0 = (int)fy;
  const int y1 = y0 + (y0 < H - 1 ? 1 : 0);
  const float ly = fy - (float)y0, hy = 1.0f - ly;
  const int64_t o0 = ((int64_t)b * H + y0) * W * C, o1 = ((int64_t)b * H + y1) * W * C;
  // four channels of source row r (0: y0, 1: y1) at element offset off
  auto ld = [&](int r, int64_t off) -> fx4 {
    const int64_t e = (r ? o1 : o0) + off;
    if constexpr (IN_BF16) {
      const uint64_t u = *(const uint64_t*)((const __bf16*)x + e);
      const uint32_t w0 = (uint32_t)u, w1 = (uint32_t)(u >> 32);
      return mk4(__uint_as_float(w0 << 16), __uint_as_float(w0 & 0xffff0000u),
                 __uint_as_float(w1 << 16), __uint_as_float(w1 & 0xffff0000u));
    } else {
      return *(const fx4*)(x + e);
    }
  };
  float* yrow = y + (int64_t)row * Wo * C;
  // the bilinear blend of the four source values
  auto blend = [&](const fx4& a, const fx4& bq, const fx4& cq, const fx4& d, float lx, float hx) {
    fx4 o;
    o.x = hy * (hx * a.x + lx * bq.x) + ly * (hx * cq.x + lx * d.x);
    o.y = hy * (hx * a.y + lx * bq.y) + ly * (hx * cq.y + lx * d.y);
    o.z = hy * (hx * a.z + lx * bq.z) + ly * (hx * cq.z + lx * d.z);
    o.w = hy * (hx * a.w + lx * bq.w) + ly * (hx * cq.w + lx * d.w);
    return o;
  };
  // output pixel ox, channels 4 cg .. 4 cg + 3; the output (4x the input) is
  // streamed out with non-temporal stores so it does not displace the source
  // rows that neighbouring output rows re-read
  auto store = [&](int ox, int cg, const fx4& o) {
    const int64_t oi = (int64_t)ox * C + 4 * cg;
    if constexpr (OUT_BF16) {  // round to nearest even, the conversion the bf16 GEMMs apply
      typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
      const bf16x4_t h = {(__bf16)o.x, (__bf16)o.y, (__bf16)o.z, (__bf16)o.w};
      __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, h),
                                  (uint64_t*)((__bf16*)y + (int64_t)row * Wo * C + oi));
    } else {
      __builtin_nontemporal_store(o, (fx4*)(yrow + oi));
    }
  };
  auto one = [&](int ox, int cg) {
    const float fx = sw * (float)ox;
    const int x0 = (int)fx;
    const int x1 = x0 + (x0 < W - 1 ? 1 : 0);
    const float lx = fx - (float)x0, hx = 1.0f - lx;
    const int64_t c0 = (int64_t)x0 * C + 4 * cg, c1 = (int64_t)x1 * C + 4 * cg;
    store(ox, cg, blend(ld(0, c0), ld(0, c1), ld(1, c0), ld(1, c1), lx, hx));
  };
  if (C4 <= 256) {
    const int ppi = 256 / C4;  // pixel runs per workgroup
    const int pp = (int)threadIdx.x / C4, cg = (int)threadIdx.x - pp * C4;
    if (pp >= ppi) return;
    const int xs = ox0 + pp * kUpsRun, xe = min(xs + kUpsRun, ox1);
    // the previous pixel's source columns p0 (values pa, pc in rows y0, y1)
    // and p1 (pb, pd); x0 repeats on every other pixel at this scale
    int p0 = -1, p1 = -1;
    fx4 pa = {}, pb = {}, pc = {}, pd = {};
    for (int ox = xs; ox < xe; ++ox) {
      const float fx = sw * (float)ox;
      const int x0 = (int)fx;
      const int x1 = x0 + (x0 < W - 1 ? 1 : 0);
      const float lx = fx - (float)x0, hx = 1.0f - lx;
      fx4 a, bq, cq, d;
      if (x0 == p0) {
        a = pa;
        cq = pc;
      } else if (x0 == p1) {
        a = pb;
        cq = pd;
      } else {
        a = ld(0, (int64_t)x0 * C + 4 * cg);
        cq = ld(1, (int64_t)x0 * C + 4 * cg);
      }
      if (x1 == x0) {
        bq = a;
        d = cq;
      } else if (x1 == p1) {
        bq = pb;
        d = pd;
      } else {
        bq = ld(0, (int64_t)x1 * C + 4 * cg);
        d = ld(1, (int64_t)x1 * C + 4 * cg);
      }
      p0 = x0;
      p1 = x1;
      pa = a;
      pc = cq;
      pb = bq;
      pd = d;
      store(ox, cg, blend(a, bq, cq, d, lx, hx));
    }
  } else {
    const int n = (ox1 - ox0) * C4;
    for (int e = (int)threadIdx.x; e < n; e += 256) {
      const int q = e / C4;
      one(ox0 + q, e - q * C4);
    }
  }
}

// 2D RoPE in place; one thread per rotated pair (token, head, axis, j < 16).
__global__ void rope2d_kernel(float* t, int32_t B, int32_t N, int32_t H, int64_t ld,
                              int32_t grid_w, const float* __restrict__ cos_t,
                              const float* __restrict__ sin_t) {
#pragma clang fp contract(off)
  const int64_t total = (int64_t)B * N * H * 32;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int j = (int)(id & 15);
  const int ax = (int)((id >> 4) & 1);
  const int64_t rest = id >> 5;
  const int h = (int)(rest % H);
  const int64_t tokg = rest / H;
  const int n = (int)(tokg % N);
  const int pos = ax ? n % grid_w : n / grid_w;
  float* u = t + tokg * ld + h * 64 + ax * 32;
  const float c = cos_t[pos * 16 + j], s = sin_t[pos * 16 + j];
  const float a = u[j], b = u[j + 16];
  u[j] = a * c - b * s;
  u[j + 16] = b * c + a * s;
}

// Token-level RoPE of MASt3REncoderV2#apply_rope (src/mastr/encoder_v2.cr:
// 204-254) with an explicit grid; one thread per element.
__global__ void rope_ref_token_kernel(const float* __restrict__ x, float* __restrict__ y,
                                      int32_t B, int32_t gh, int32_t gw, int32_t D,
                                      int32_t hd, const float* __restrict__ cos_t,
                                      const float* __restrict__ sin_t) {
  const int64_t total = (int64_t)B * gh * gw * D;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int d = (int)(id % D);
  const int64_t tok = id / D;
  const int n = (int)(tok % ((int64_t)gh * gw));
  const int yy = n / gw, xi = n - yy * gw;
  const int half = hd / 2, dh = d % hd;
  if (dh < half) {
    const float c = cos_t[yy * half + dh], s = sin_t[yy * half + dh];
    y[id] = x[id] * c - x[id + half] * s;
  } else {
    const int f = dh - half;
    const float c = cos_t[xi * half + f], s = sin_t[xi * half + f];
    y[id] = x[id - half] * s + x[id] * c;
  }
}

// DPT head tail: 1x1 conv Cin -> 4 (+bias), pts = ch 0..2, conf = 1 + exp(ch 3)
// (the reference's split_output, src/mastr/decoder_v2.cr:619-655, with the
// MASt3R confidence mapping) or, SIGMOID, the reference's own 1 / (1 + exp(-x)).
constexpr int kHeadOutIter = 8;  // groups of 32 pixels per workgroup

// INH: x holds bf16 (the bf16 mode's head.2 writes its ReLU output so); a
// lane's 16-byte chunks then hold 8 channels.
template <bool SIGMOID, bool INH>
__global__ __launch_bounds__(256) void head_out_kernel(const float* __restrict__ x, int64_t P,
                                                       int32_t Cin, const float* __restrict__ w,
                                                       const float* __restrict__ b,
                                                       float* __restrict__ pts,
                                                       float* __restrict__ conf) {
  // Eight lanes share one pixel: lane `sub` reads the 16-byte channel chunks
  // sub, sub + 8, ..., so each load instruction covers whole 128-byte lines of
  // eight pixels. The four dot products are then summed over the eight lanes.
  extern __shared__ float ws[];  // [4][Cin]
  for (int i = threadIdx.x; i < 4 * Cin; i += blockDim.x) ws[i] = w[i];
  __syncthreads();
  const int sub = threadIdx.x & 7;
  const int n4 = Cin >> 2;
  const fx4* w0 = (const fx4*)ws;
  const fx4* w1 = w0 + n4;
  const fx4* w2 = w1 + n4;
  const fx4* w3 = w2 + n4;
  for (int it = 0; it < kHeadOutIter; ++it) {
    const int64_t px = ((int64_t)blockIdx.x * kHeadOutIter + it) * 32 + (threadIdx.x >> 3);
    if (px >= P) break;  // uniform within each group of eight lanes
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    auto dot4 = [&](const fx4& v, int c4) {
      const fx4 q0 = w0[c4], q1 = w1[c4], q2 = w2[c4], q3 = w3[c4];
      a0 += v.x * q0.x + v.y * q0.y + v.z * q0.z + v.w * q0.w;
      a1 += v.x * q1.x + v.y * q1.y + v.z * q1.z + v.w * q1.w;
      a2 += v.x * q2.x + v.y * q2.y + v.z * q2.z + v.w * q2.w;
      a3 += v.x * q3.x + v.y * q3.y + v.z * q3.z + v.w * q3.w;
    };
    if constexpr (INH) {
      typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
      const u32x4_t* xr = (const u32x4_t*)((const __bf16*)x + px * Cin);
      auto lo = [](uint32_t u) { return __uint_as_float(u << 16); };
      auto hi = [](uint32_t u) { return __uint_as_float(u & 0xffff0000u); };
#pragma unroll 2
      for (int c8 = sub; c8 < (n4 >> 1); c8 += 8) {
        const u32x4_t u = xr[c8];
        dot4(mk4(lo(u.x), hi(u.x), lo(u.y), hi(u.y)), 2 * c8);
        dot4(mk4(lo(u.z), hi(u.z), lo(u.w), hi(u.w)), 2 * c8 + 1);
      }
    } else {
      const fx4* xr = (const fx4*)(x + px * Cin);
#pragma unroll 4
      for (int c4 = sub; c4 < n4; c4 += 8) dot4(xr[c4], c4);
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {  // xor 1, 2, 4 stay inside the group
      a0 += __shfl_xor(a0, o);
      a1 += __shfl_xor(a1, o);
      a2 += __shfl_xor(a2, o);
      a3 += __shfl_xor(a3, o);
    }
    if (sub < 3) {
      pts[px * 3 + sub] = (sub == 0 ? a0 : sub == 1 ? a1 : a2) + b[sub];
    } else if (sub == 3) {
      const float raw = a3 + b[3];
      conf[px] = SIGMOID ? 1.0f / (1.0f + expf(-raw)) : 1.0f + expf(raw);
    }
  }
}

inline unsigned nblocks(int64_t total, int per) { return (unsigned)((total + per - 1) / per); }
// A 1-D grid of `per` items per block must fit grid.x (callers check this
// before nblocks, so negative sizes and wrapped block counts become errors).
inline bool grid_fits(int64_t total, int per) { return total >= 0 && total / per < INT32_MAX; }
bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

int launch_layernorm(const LnBatch& bt, hipStream_t s) {
  GS_REQUIRE(bt.ngroups >= 1 && bt.ngroups <= kMaxGroups, "layernorm: bad group count");
  int64_t max_rows = 0;
  const int D = bt.g[0].D;
  for (int i = 0; i < bt.ngroups; ++i) {
    const LnArgs& a = bt.g[i];
    GS_REQUIRE(a.D == D, "layernorm: grouped rows must share D");
    GS_REQUIRE(a.x && (a.y || a.stats) && a.gamma && a.beta, "layernorm: null operand");
    GS_REQUIRE(aligned16(a.x) && (!a.y || aligned16(a.y)) && aligned16(a.gamma) &&
                   aligned16(a.beta),
               "layernorm: operands must be 16-byte aligned");
    max_rows = a.rows > max_rows ? a.rows : max_rows;
  }
  GS_REQUIRE(D > 0 && D % 4 == 0 && D <= 4096, "layernorm: need 0 < D <= 4096, D % 4 == 0");
  if (max_rows == 0) return 0;
  dim3 grid(std::min(nblocks(max_rows, 4), (unsigned)kLnBlocks), bt.ngroups), block(256);
  hipEvent_t ev = prof_start(s);
  if (D <= 1024)
    hipLaunchKernelGGL(layernorm_kernel<4>, grid, block, 0, s, bt);
  else
    hipLaunchKernelGGL(layernorm_kernel<16>, grid, block, 0, s, bt);
  GS_CHECK_HIP(hipGetLastError());
  if (ev) {
    double rows = 0, bytes = 0;
    for (int i = 0; i < bt.ngroups; ++i) {
      rows += (double)bt.g[i].rows;
      const double per = !bt.g[i].y ? 4.0 : (bt.g[i].y_bf16 ? 6.0 : 8.0);  // stats-only: read
      bytes += per * (double)bt.g[i].rows * D + 8.0 * D + (bt.g[i].stats ? 8.0 * bt.g[i].rows : 0.0);
    }
    prof_stop(s, ev, "layernorm_kernel", 8.0 * rows * D, bytes);
  }
  return 0;
}

int launch_unfold(const float* img, int32_t B, int32_t H, int32_t W, int32_t p,
                  float* out, hipStream_t s) {
  GS_REQUIRE(p > 0 && p % 4 == 0 && H % p == 0 && W % p == 0,
             "unfold: H, W must be multiples of p, p % 4 == 0");
  GS_REQUIRE(aligned16(img) && aligned16(out), "unfold: operands must be 16-byte aligned");
  const int64_t total = (int64_t)B * (H / p) * (W / p) * (3 * p * p / 4);
  GS_REQUIRE(B >= 0 && H >= 0 && W >= 0 && grid_fits(total, 256), "unfold: bad sizes");
  if (total == 0) return 0;
  hipEvent_t ev = prof_start(s);
  hipLaunchKernelGGL(unfold_kernel, dim3(nblocks(total, 256)), dim3(256), 0, s, img, B, H, W,
                     p, out);
  GS_CHECK_HIP(hipGetLastError());
  prof_stop(s, ev, "unfold_kernel", 0.0, 8.0 * (double)total * 4.0);
  return 0;
}

int launch_upsample2x(const float* x, int32_t B, int32_t H, int32_t W, int32_t C,
                      float* y, hipStream_t s, bool out_bf16, bool in_bf16) {
  GS_REQUIRE(C > 0 && C % 4 == 0 && H > 0 && W > 0 && B >= 0, "upsample2x: need C % 4 == 0");
  GS_REQUIRE(aligned16(x) && aligned16(y), "upsample2x: operands must be 16-byte aligned");
  GS_REQUIRE((int64_t)2 * W * (C / 4) <= INT32_MAX && (int64_t)2 * B * H <= INT32_MAX,
             "upsample2x: too many elements");
  // pixels per workgroup: 256 / (C / 4) runs of kUpsRun pixels, or eight
  // pixels of wider rows
  const int32_t px = C / 4 <= 256 ? kUpsRun * (256 / (C / 4)) : 8;
  const int32_t blocks_per_row = (int32_t)nblocks((int64_t)2 * W, px);
  const int64_t nblk = (int64_t)2 * B * H * blocks_per_row;
  GS_REQUIRE(nblk < INT32_MAX, "upsample2x: too many elements");
  if (nblk == 0) return 0;
  hipEvent_t ev = prof_start(s);
  const dim3 grid((uint32_t)nblk), block(256);
  if (in_bf16 && out_bf16)
    hipLaunchKernelGGL((upsample2x_kernel<true, true>), grid, block, 0, s, x, H, W, C, blocks_per_row,
                       px, y);
  else if (in_bf16)
    hipLaunchKernelGGL((upsample2x_kernel<true, false>), grid, block, 0, s, x, H, W, C,
                       blocks_per_row, px, y);
  else if (out_bf16)
    hipLaunchKernelGGL((upsample2x_kernel<false, true>), grid, block, 0, s, x, H, W, C,
                       blocks_per_row, px, y);
  else
    hipLaunchKernelGGL((upsample2x_kernel<false, false>), grid, block, 0, s, x, H, W, C,
                       blocks_per_row, px, y);
  GS_CHECK_HIP(hipGetLastError());
  prof_stop(s, ev, "upsample2x_kernel", 0.0,
            (double)B * H * W * C * ((in_bf16 ? 2.0 : 4.0) + (out_bf16 ? 8.0 : 16.0)));
  return 0;
}

int launch_rope2d(float* t, int32_t B, int32_t N, int32_t H, int64_t ld, int32_t grid_w,
                  const float* cos_t, const float* sin_t, hipStream_t s) {
  GS_REQUIRE(t && B >= 0 && N >= 0 && H > 0 && ld >= (int64_t)H * 64 && grid_w > 0,
             "rope2d: bad layout");
  const int64_t total = (int64_t)B * N * H * 32;
  GS_REQUIRE(grid_fits(total, 256), "rope2d: too many elements");
  if (total == 0) return 0;
  hipLaunchKernelGGL(rope2d_kernel, dim3(nblocks(total, 256)), dim3(256), 0, s, t, B, N, H,
                     ld, grid_w, cos_t, sin_t);
  GS_CHECK_HIP(hipGetLastError());
  return 0;
}

int launch_rope_ref_token(const float* x, float* y, int32_t B, int32_t gh, int32_t gw,
                          int32_t D, int32_t H, const float* cos_t, const float* sin_t,
                          int32_t max_pos, hipStream_t s) {
  GS_REQUIRE(H > 0 && D % H == 0 && (D / H) % 2 == 0, "rope_ref_token: bad head split");
  GS_REQUIRE(gh <= max_pos && gw <= max_pos, "rope_ref_token: table too small");
  GS_REQUIRE(B >= 0 && gh >= 0 && gw >= 0 && D > 0, "rope_ref_token: bad sizes");
  const int64_t total = (int64_t)B * gh * gw * D;
  GS_REQUIRE(grid_fits(total, 256), "rope_ref_token: too many elements");
  if (total == 0) return 0;
  hipLaunchKernelGGL(rope_ref_token_kernel, dim3(nblocks(total, 256)), dim3(256), 0, s, x, y,
                     B, gh, gw, D, D / H, cos_t, sin_t);
  GS_CHECK_HIP(hipGetLastError());
  return 0;
}

int launch_head_out(const float* x, int64_t P, int32_t Cin, const float* w, const float* b,
                    float* pts, float* conf, bool sigmoid, hipStream_t s, bool in_bf16) {
  GS_REQUIRE(Cin % 4 == 0 && Cin <= 4096, "head_out: need Cin % 4 == 0");
  GS_REQUIRE(!in_bf16 || Cin % 8 == 0, "head_out: bf16 input needs Cin % 8 == 0");
  GS_REQUIRE(aligned16(x), "head_out: input must be 16-byte aligned");
  GS_REQUIRE(grid_fits(P, 32 * kHeadOutIter), "head_out: bad pixel count");
  if (P == 0) return 0;
  hipEvent_t ev = prof_start(s);
  const dim3 grid(nblocks(P, 32 * kHeadOutIter)), block(256);
  const size_t lds = 4 * Cin * sizeof(float);
  if (sigmoid && in_bf16)
    hipLaunchKernelGGL((head_out_kernel<true, true>), grid, block, lds, s, x, P, Cin, w, b, pts, conf);
  else if (sigmoid)
    hipLaunchKernelGGL((head_out_kernel<true, false>), grid, block, lds, s, x, P, Cin, w, b, pts, conf);
  else if (in_bf16)
    hipLaunchKernelGGL((head_out_kernel<false, true>), grid, block, lds, s, x, P, Cin, w, b, pts, conf);
  else
    hipLaunchKernelGGL((head_out_kernel<false, false>), grid, block, lds, s, x, P, Cin, w, b, pts, conf);
  GS_CHECK_HIP(hipGetLastError());
  prof_stop(s, ev, "head_out_kernel", 8.0 * (double)P * Cin,
            (in_bf16 ? 2.0 : 4.0) * (double)P * Cin + 16.0 * (double)P);
  return 0;
}

void rope_table_host(int32_t max_pos, float base, float* cos_t, float* sin_t) {
  // inv_freq_j = 1 / base^(2j/32) for the 16 frequency pairs of one 32-dim
  // axis half; theta = pos * inv_freq_j in fp32, libm cos/sin.
  for (int32_t p = 0; p < max_pos; ++p)
    for (int32_t j = 0; j < 16; ++j) {
      const float inv = 1.0f / powf(base, (float)(2 * j) / 32.0f);
      const float th = (float)p * inv;
      cos_t[p * 16 + j] = cosf(th);
      sin_t[p * 16 + j] = sinf(th);
    }
}

void rope_ref_table_host(int32_t max_pos, int32_t hd, float base, float* cos_t,
                         float* sin_t) {
  const int32_t half = hd / 2;
  for (int32_t p = 0; p < max_pos; ++p)
    for (int32_t i = 0; i < half; ++i) {
      const float f = 1.0f / powf(base, (2.0f * (float)i) / (float)hd);
      const float th = (float)p * f;
      cos_t[p * half + i] = cosf(th);
      sin_t[p * half + i] = sinf(th);
    }
}

}  // namespace gs

namespace gs {
namespace {

__global__ void oihw_to_ohwi_kernel(const float* __restrict__ w, int32_t Cout, int32_t Cin,
                                    int32_t k, float* __restrict__ out) {
  const int64_t total = (int64_t)Cout * Cin * k * k;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  // id indexes the OHWI output: ((oc*k + kh)*k + kw)*Cin + ic
  const int ic = (int)(id % Cin);
  int64_t r = id / Cin;
  const int kw = (int)(r % k);
  r /= k;
  const int kh = (int)(r % k);
  const int oc = (int)(r / k);
  out[id] = w[(((int64_t)oc * Cin + ic) * k + kh) * k + kw];
}

__global__ void convt_relayout_kernel(const float* __restrict__ w, const float* __restrict__ b,
                                      int32_t Cin, int32_t Cout, int32_t k,
                                      float* __restrict__ wout, float* __restrict__ bout) {
  const int64_t N = (int64_t)k * k * Cout;
  const int64_t total = N * Cin;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int ic = (int)(id % Cin);
  const int64_t n = id / Cin;
  const int oc = (int)(n % Cout);
  const int ij = (int)(n / Cout);
  const int i = ij / k, j = ij - i * k;
  wout[id] = w[(((int64_t)ic * Cout + oc) * k + i) * k + j];
  if (ic == 0 && bout) bout[n] = b ? b[oc] : 0.f;
}

}  // namespace

int launch_oihw_to_ohwi(const float* w, int32_t Cout, int32_t Cin, int32_t k, float* out,
                        hipStream_t s) {
  const int64_t total = (int64_t)Cout * Cin * k * k;
  if (total == 0) return 0;
  hipLaunchKernelGGL(oihw_to_ohwi_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     s, w, Cout, Cin, k, out);
  GS_CHECK_HIP(hipGetLastError());
  return 0;
}

int launch_convt_relayout(const float* w, const float* b, int32_t Cin, int32_t Cout, int32_t k,
                          float* wout, float* bout, hipStream_t s) {
  const int64_t total = (int64_t)k * k * Cout * Cin;
  if (total == 0) return 0;
  hipLaunchKernelGGL(convt_relayout_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     s, w, b, Cin, Cout, k, wout, bout);
  GS_CHECK_HIP(hipGetLastError());
  return 0;
}

}  // namespace gs

namespace gs {
namespace {

// fp32 -> bf16, round to nearest even (the weight copies of the bf16 path).
__global__ void f32_to_bf16_kernel(const float* __restrict__ in, __bf16* __restrict__ out,
                                   int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 3 < n) {
    const fx4 v = *(const fx4*)(in + i);
    out[i] = (__bf16)v.x;
    out[i + 1] = (__bf16)v.y;
    out[i + 2] = (__bf16)v.z;
    out[i + 3] = (__bf16)v.w;
  } else {
    for (int64_t j = i; j < n; ++j) out[j] = (__bf16)in[j];
  }
}

// Exact three-term bf16 split (x0 = bf16(x), x1 = bf16(x - x0), x2 =
// bf16(x - x0 - x1)), the same arithmetic as the bf16x6 GEMM's on-the-fly
// split, so pre-split weights give bit-identical products.
__global__ void f32_to_bf16x3_kernel(const float* __restrict__ in, __bf16* __restrict__ out,
                                     int64_t n, int64_t plane) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = in[i];
  const __bf16 h = (__bf16)v;
  const float r1 = v - (float)h;
  const __bf16 m = (__bf16)r1;
  const float r2 = r1 - (float)m;
  out[i] = h;
  out[plane + i] = m;
  out[2 * plane + i] = (__bf16)r2;
}

}  // namespace

int launch_f32_to_bf16x3(const float* in, void* out, int64_t n, int64_t plane, hipStream_t s) {
  if (n <= 0) return 0;
  GS_REQUIRE(in && out && plane >= n, "f32_to_bf16x3: bad arguments");
  hipLaunchKernelGGL(f32_to_bf16x3_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in,
                     (__bf16*)out, n, plane);
  GS_CHECK_HIP(hipGetLastError());
  return 0;
}

int launch_f32_to_bf16(const float* in, void* out, int64_t n, hipStream_t s) {
  if (n <= 0) return 0;
  GS_REQUIRE(((uintptr_t)in & 15) == 0, "f32_to_bf16: input must be 16-byte aligned");
  const int64_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                     in, (__bf16*)out, n);
  GS_CHECK_HIP(hipGetLastError());
  return 0;
}

}  // namespace gs
