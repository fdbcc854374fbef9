// Caller-side passes around the pair path, on the device:
//   image_prep_kernel   resize_image (src/mastr/inference.cr:330-374) and
//                       preprocess_image (193-229), separately or fused;
//   cp_*_kernel         collect_points (296-328) as an order-preserving
//                       stream compaction (count, scan, scatter).
// All three are HBM-bound byte movers: no MFMA, coalesced rows, one pass each.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/gs_hip.h"
#include "internal.h"

#pragma clang fp contract(off)  // fp32 sequences as the reference evaluates them

namespace gs {
namespace {

constexpr int kCpThreads = 256;
constexpr int kCpPer = 16;
constexpr int kCpTile = kCpThreads * kCpPer;  // confidences per block

// One thread per output pixel (all channels). RESIZE: bilinear with the
// reference's fp32 source coordinate (ty * (sh-1)) / (th-1), truncation and
// clamp to [0, s-2], four-term sum in the reference's order. NORM: ImageNet
// (v - mean) / std (C == 3). NCHW: planar output, else interleaved.
template <bool RESIZE, bool NORM, bool NCHW>
__global__ __launch_bounds__(256) void image_prep_kernel(const float* __restrict__ src,
                                                         int64_t total, int32_t sh, int32_t sw,
                                                         int32_t C, int32_t th, int32_t tw,
                                                         float* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int32_t tx = (int32_t)(i % tw);
  const int64_t r = i / tw;
  const int32_t ty = (int32_t)(r % th);
  const int64_t f = r / th;
  const float* img = src + f * sh * sw * C;
  const float mean[3] = {0.485f, 0.456f, 0.406f};
  const float stdv[3] = {0.229f, 0.224f, 0.225f};
  int64_t i00 = ((int64_t)ty * sw + tx) * C, i01 = 0, i10 = 0, i11 = 0;
  float fy = 0.f, fx = 0.f;
  if (RESIZE) {
    const float sy = (float)ty * (float)(sh - 1) / (float)(th - 1);
    const float sx = (float)tx * (float)(sw - 1) / (float)(tw - 1);
    const int32_t y0 = min(max((int32_t)sy, 0), sh - 2);
    const int32_t x0 = min(max((int32_t)sx, 0), sw - 2);
    fy = sy - (float)y0;
    fx = sx - (float)x0;
    i00 = ((int64_t)y0 * sw + x0) * C;
    i01 = i00 + C;
    i10 = i00 + (int64_t)sw * C;
    i11 = i10 + C;
  }
  for (int32_t c = 0; c < C; ++c) {
    float v;
    if (RESIZE) {
      v = img[i00 + c] * (1 - fx) * (1 - fy) + img[i01 + c] * fx * (1 - fy) +
          img[i10 + c] * (1 - fx) * fy + img[i11 + c] * fx * fy;
    } else {
      v = img[i00 + c];
    }
    if (NORM) v = (v - mean[c]) / stdv[c];
    if (NCHW)
      dst[((f * C + c) * th + ty) * tw + tx] = v;
    else
      dst[(r * tw + tx) * C + c] = v;
  }
}

__device__ __forceinline__ int block_sum_256(int v, int* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  const int t = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return t;
}

// Pass 1: selected count of each kCpTile-confidence block.
__global__ __launch_bounds__(kCpThreads) void cp_count_kernel(const float* __restrict__ conf,
                                                              int64_t n, float thr,
                                                              int64_t* __restrict__ blk) {
  __shared__ int red[4];
  const int64_t base = (int64_t)blockIdx.x * kCpTile;
  int cnt = 0;
#pragma unroll
  for (int k = 0; k < kCpPer; ++k) {
    const int64_t e = base + k * kCpThreads + threadIdx.x;
    if (e < n && conf[e] > thr) ++cnt;
  }
  const int t = block_sum_256(cnt, red);
  if (threadIdx.x == 0) blk[blockIdx.x] = t;
}

// Pass 2 (one workgroup): exclusive scan of the block counts, offset by the
// running total in *counter, which is then advanced by this call's total.
__global__ __launch_bounds__(1024) void cp_scan_kernel(int64_t* __restrict__ blk, int64_t nblk,
                                                       int64_t* __restrict__ counter) {
  __shared__ int64_t wsum[16];
  __shared__ int64_t s_base;
  if (threadIdx.x == 0) s_base = counter[0];
  __syncthreads();
  int64_t running = s_base;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int64_t j0 = 0; j0 < nblk; j0 += 1024) {
    const int64_t j = j0 + threadIdx.x;
    const int64_t v = j < nblk ? blk[j] : 0;
    int64_t incl = v;  // inclusive wave scan
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t u = __shfl_up(incl, o);
      if (lane >= o) incl += u;
    }
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    int64_t before = 0, chunk = 0;
    for (int q = 0; q < 16; ++q) {
      if (q < w) before += wsum[q];
      chunk += wsum[q];
    }
    if (j < nblk) blk[j] = running + before + incl - v;
    running += chunk;
    __syncthreads();  // wsum reused by the next chunk
  }
  if (threadIdx.x == 0) counter[0] = running;
}

// Pass 3: order-preserving scatter. Round k of a block covers confidences
// base + k*256 + [0, 256): a wave ballot ranks the selected lanes, wave
// totals in LDS rank the waves.
__global__ __launch_bounds__(kCpThreads) void cp_scatter_kernel(
    const float* __restrict__ pts, const float* __restrict__ conf, int64_t n, float thr,
    const int64_t* __restrict__ blk, float* __restrict__ out_pts, float* __restrict__ out_conf,
    int64_t cap) {
  __shared__ int wtot[kCpPer][4];
  const int64_t base = (int64_t)blockIdx.x * kCpTile;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  bool sel[kCpPer];
  float cv[kCpPer];
  int rank[kCpPer];
#pragma unroll
  for (int k = 0; k < kCpPer; ++k) {
    const int64_t e = base + k * kCpThreads + threadIdx.x;
    cv[k] = e < n ? conf[e] : 0.f;
    sel[k] = e < n && cv[k] > thr;
    const uint64_t m = __ballot(sel[k]);
    rank[k] = __popcll(m & below);
    if (lane == 0) wtot[k][w] = __popcll(m);
  }
  __syncthreads();
  int64_t off = blk[blockIdx.x];
#pragma unroll
  for (int k = 0; k < kCpPer; ++k) {
    int before = 0;
    for (int q = 0; q < w; ++q) before += wtot[k][q];
    const int64_t pos = off + before + rank[k];
    if (sel[k] && pos < cap) {
      const int64_t e = base + k * kCpThreads + threadIdx.x;
      out_pts[3 * pos] = pts[3 * e];
      out_pts[3 * pos + 1] = pts[3 * e + 1];
      out_pts[3 * pos + 2] = pts[3 * e + 2];
      out_conf[pos] = cv[k];
    }
    off += wtot[k][0] + wtot[k][1] + wtot[k][2] + wtot[k][3];
  }
}

unsigned grid_for(int64_t total) { return (unsigned)((total + 255) / 256); }

__global__ void fill_i64_kernel(int64_t* p, int64_t n, int64_t v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

int launch_image_prep(const float* src, int32_t F, int32_t sh, int32_t sw, int32_t C,
                      int32_t th, int32_t tw, bool resize, bool normalize, bool nchw,
                      float* dst, hipStream_t s) {
  GS_REQUIRE(F >= 0 && C > 0 && sh > 0 && sw > 0 && th > 0 && tw > 0,
             "image_prep: bad sizes");
  GS_REQUIRE(!resize || (sh >= 2 && sw >= 2 && th >= 2 && tw >= 2),
             "resize_image: source and target sides must be >= 2");
  GS_REQUIRE(resize || (sh == th && sw == tw), "image_prep: size change needs resize");
  GS_REQUIRE(!normalize || C == 3, "preprocess_image: needs 3 channels");
  GS_REQUIRE(src && dst, "image_prep: null pointer");
  const int64_t total = (int64_t)F * th * tw;
  if (total == 0) return 0;
  GS_REQUIRE(total / 256 < INT32_MAX, "image_prep: too many pixels");
  hipEvent_t ev = prof_start(s);
  const dim3 grid(grid_for(total)), blk(256);
  const char* name;
#define GS_PREP(R, N, P)                                                                   \
  hipLaunchKernelGGL((image_prep_kernel<R, N, P>), grid, blk, 0, s, src, total, sh, sw, C, \
                     th, tw, dst)
  if (resize && normalize && nchw) {
    GS_PREP(true, true, true);
    name = "image_prep_kernel<resize,norm,nchw>";
  } else if (resize && !normalize && !nchw) {
    GS_PREP(true, false, false);
    name = "image_prep_kernel<resize>";
  } else if (!resize && normalize && nchw) {
    GS_PREP(false, true, true);
    name = "image_prep_kernel<norm,nchw>";
  } else {
    GS_REQUIRE(false, "image_prep: unsupported combination");
  }
#undef GS_PREP
  GS_CHECK_HIP(hipGetLastError());
  const double src_bytes = resize ? 4.0 * (double)F * sh * sw * C : 4.0 * (double)total * C;
  prof_stop(s, ev, name, 0.0, src_bytes + 4.0 * (double)total * C);
  return 0;
}

int64_t collect_points_scratch(int64_t n) { return (n + kCpTile - 1) / kCpTile; }

int launch_collect_points(const float* pts, const float* conf, int64_t n, float thr,
                          float* out_pts, float* out_conf, int64_t cap, int64_t* counter,
                          int64_t* scratch, hipStream_t s) {
  GS_REQUIRE(n >= 0 && cap >= 0 && counter, "collect_points: bad arguments");
  GS_REQUIRE(cap == 0 || (out_pts && out_conf), "collect_points: null output");
  if (n == 0) return 0;
  GS_REQUIRE(pts && conf && scratch, "collect_points: null input");
  const int64_t nblk = collect_points_scratch(n);
  GS_REQUIRE(nblk <= INT32_MAX, "collect_points: too many points");
  hipEvent_t ev = prof_start(s);
  hipLaunchKernelGGL(cp_count_kernel, dim3((uint32_t)nblk), dim3(kCpThreads), 0, s, conf, n, thr,
                     scratch);
  hipLaunchKernelGGL(cp_scan_kernel, dim3(1), dim3(1024), 0, s, scratch, nblk, counter);
  hipLaunchKernelGGL(cp_scatter_kernel, dim3((uint32_t)nblk), dim3(kCpThreads), 0, s, pts, conf,
                     n, thr, scratch, out_pts, out_conf, cap);
  GS_CHECK_HIP(hipGetLastError());
  // bytes with every point selected: confidences read twice, points read,
  // points and confidences written (36 B per point; an upper bound otherwise)
  prof_stop(s, ev, "collect_points", 0.0, 36.0 * (double)n);
  return 0;
}

int launch_fill_i64(int64_t* p, int64_t n, int64_t v, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(fill_i64_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n, v);
  GS_CHECK_HIP(hipGetLastError());
  return 0;
}

}  // namespace gs

// ---- compaction without allocation ----------------------------------------------
// gs_hip_collect_points_noalloc keeps its block counts in `scratch`, a
// file-scope device array: every GPU the library runs on holds its own copy
// (256 KB) until the process ends. In host code the array's name is only a
// stand-in; its device address on the current device comes from
// hipGetSymbolAddress, looked up once per device and used for every launch.
// The count pass writes every block count the scan then reads, so the array
// needs no clearing between calls.
namespace gs {
namespace {
constexpr int64_t kNoAllocMaxPoints = (int64_t)1 << 27;
constexpr int64_t kNoAllocBlocks = kNoAllocMaxPoints / kCpTile;
static_assert(kNoAllocMaxPoints % kCpTile == 0, "whole blocks");
}  // namespace
}  // namespace gs

static __device__ __align__(256) int64_t scratch[gs::kNoAllocBlocks];

namespace gs {
namespace {
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
int64_t* g_noalloc_ptr[kNoAllocMaxDevices] = {};

int noalloc_scratch(int64_t** out) {
  int dev = 0;
  GS_CHECK_HIP(hipGetDevice(&dev));
  GS_REQUIRE(dev >= 0 && dev < kNoAllocMaxDevices, "collect_points_noalloc: device out of range");
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    GS_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    GS_REQUIRE(p != nullptr, "collect_points_noalloc: no device address for the scratch array");
    g_noalloc_ptr[dev] = (int64_t*)p;
  }
  *out = g_noalloc_ptr[dev];
  return 0;
}
}  // namespace
}  // namespace gs

extern "C" int32_t gs_hip_collect_points_noalloc(const float* pts, const float* conf, int64_t n,
                                                 float threshold, float* out_pts,
                                                 float* out_conf, int64_t capacity,
                                                 int64_t* count, void* stream) {
  if (gs::ensure_device()) return -2;
  GS_REQUIRE(n >= 0 && n <= gs::kNoAllocMaxPoints,
             "collect_points_noalloc: n must be in [0, 2^27] (134217728 points)");
  int64_t* sc = nullptr;
  if (n > 0) {
    const int rc = gs::noalloc_scratch(&sc);
    if (rc) return rc;
  }
  return gs::launch_collect_points(pts, conf, n, threshold, out_pts, out_conf, capacity, count, sc,
                                   (hipStream_t)stream);
}
