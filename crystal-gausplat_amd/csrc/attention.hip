// Flash attention (online softmax) on gfx950 matrix cores, fp32, head dim 64.
//
// Replaces the reference's attention paths: the CPU loops of
// MultiHeadAttention#scaled_dot_product_attention_cpu
// (src/nn/attention.cr:215-325: scores, row max, exp, sum, divide, P.V) and the
// Metal flash_attention kernel behind GPUOps.fused_attention
// (src/nn/gpu_ops.cr:200-227). Self and cross attention (Nq != Nkv allowed).
//
// Workgroup = 4 wavefronts = 128 queries of one (batch, head). K/V tiles of
// 64 keys are staged through LDS (shared by the 4 wavefronts) and prefetched
// into registers one tile ahead. Each wavefront computes, per 32-key block:
//   S^T (32 keys x 32 queries) = K . Q^T   -- 32 x v_mfma_f32_32x32x2_f32
//   O^T (64 x 32)             += V^T . P^T -- 2 x 16 MFMAs
// Computing S transposed puts all 16 scores a lane holds in one query column
// (query = lane % 32), so the row max / row sum need one cross-half exchange
// and the exponentiated scores are already the B operand of the P.V product:
// MFMA step s takes key 8*(s/4) + 4*(lane/32) + s%4 -- exactly the key the
// lane holds in accumulator register s. No LDS round trip for P.
// The exponentials are the hardware exp2 (v_exp_f32, one instruction): it
// flushes results below 2^-126 to zero, i.e. it drops only terms that are
// 2^-126 below the running row maximum (exp2(-inf) = 0 for masked keys and
// for the first rescale).
#include <string>
#include <type_traits>

#include "bf16_split.h"
#include "internal.h"

typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace gs {
namespace {

constexpr int QT = 128;  // queries per workgroup
constexpr int KT = 64;   // keys per LDS tile
constexpr int HD = 64;
constexpr int kAttnCUs = 256;  // MI355X compute units

// Workgroups go to the 8 XCDs round-robin by linear id, and each XCD has its
// own L2. The logical (query tile, head, image) of a workgroup is therefore
// taken from a remapped id that gives every XCD one contiguous range of the
// x-fastest order: the query tiles of one (image, head) run on one XCD at
// about the same time and read its K / V through one L2, instead of every
// XCD fetching them. XCD c (of 8) runs logical ids
// [c*q + min(c, r), ... + q + (c < r)), q = total / 8, r = total % 8.
struct AttnTile {
  int x, y, z;
};
__device__ __forceinline__ AttnTile attn_tile() {
  const int64_t gx = gridDim.x, gy = gridDim.y;
  const int64_t total = gx * gy * (int64_t)gridDim.z;
  const int64_t L = blockIdx.x + gx * (blockIdx.y + gy * (int64_t)blockIdx.z);
  const int64_t q = total >> 3, r = total & 7, c = L & 7;
  const int64_t w = c * q + (c < r ? c : r) + (L >> 3);
  const int64_t yz = w / gx;
  return AttnTile{(int)(w - yz * gx), (int)(yz % gy), (int)(yz / gy)};
}

// SPLIT: workgroup (query tile, key range) = (x / kv_split, x % kv_split) of
// its remapped tile processes keys [range * kv_chunk, + kv_chunk) and
// writes its unnormalised output with the running max and sum to the
// scratch; attn_merge_kernel combines the ranges.
template <bool SPLIT>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttnBatch batch, int32_t Bcount) {
  constexpr int NW = 4, KTT = KT, KP = KTT / (4 * NW);  // K/V fx4 loads per thread per tile
  const AttnTile tile = attn_tile();
  const int grp = tile.z / Bcount;
  const int b = tile.z - grp * Bcount;
  const AttnArgs& p = batch.g[grp];
  const int head = tile.y;
  const int Nq = p.Nq, Nkv = p.Nkv;

  __shared__ __attribute__((aligned(16))) float Ks[KTT][HD + 4];
  __shared__ __attribute__((aligned(16))) float Vs[KTT][HD];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;

  const float* qb = p.q + (int64_t)b * p.q_sb + (int64_t)head * p.q_sh;
  const float* kb = p.k + (int64_t)b * p.k_sb + (int64_t)head * p.k_sh;
  const float* vb = p.v + (int64_t)b * p.v_sb + (int64_t)head * p.v_sh;
  float* ob = p.o + (int64_t)b * p.o_sb + (int64_t)head * p.o_sh;

  const int ns = SPLIT ? batch.kv_split : 1;
  const int qtile = SPLIT ? tile.x / ns : tile.x;
  const int krange = SPLIT ? tile.x - qtile * ns : 0;
  const int kbeg = SPLIT ? krange * batch.kv_chunk : 0;
  const int kend = SPLIT ? min(kbeg + batch.kv_chunk, Nkv) : Nkv;
  const int q0 = qtile * (32 * NW) + wave * 32;
  // Q fragment: lane holds q[query l32][32*hl .. 32*hl+31], pre-scaled so the
  // softmax runs in base 2: exp(s - m) == exp2(s*log2e - m*log2e).
  const float qscale = p.scale * 1.4426950408889634f;
  float qf[32];
  {
    const int qrow = min(q0 + l32, Nq - 1);
    const float* qr = qb + (int64_t)qrow * p.q_sn + hl * 32;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const fx4 v = *(const fx4*)(qr + 4 * t);
      qf[4 * t + 0] = v.x * qscale;
      qf[4 * t + 1] = v.y * qscale;
      qf[4 * t + 2] = v.z * qscale;
      qf[4 * t + 3] = v.w * qscale;
    }
  }

  floatx16 o0 = {}, o1 = {};
  float m_run = -INFINITY, l_run = 0.f;

  // Tile load assignment: key rows tid/16 + 4*NW*i, fx4 column tid%16. The
  // loads go through buffer resources whose base is the tile's first key row
  // and whose size ends at key kend - 1's 64 values, so the lane offsets stay
  // fixed across tiles and rows at or past kend read as zero (key rows are at
  // least HD apart and each (image, head) span is below 2 GiB, checked on the
  // host): no 64-bit address arithmetic and no range branches per tile.
  const int lrow = tid >> 4, lc4 = (tid & 15) * 4;
  fx4 rk[KP], rv[KP];
  uint32_t kvo[KP], vvo[KP];
#pragma unroll
  for (int i = 0; i < KP; ++i) {
    kvo[i] = (uint32_t)(((int64_t)(lrow + 4 * NW * i) * p.k_sn + lc4) * 4);
    vvo[i] = (uint32_t)(((int64_t)(lrow + 4 * NW * i) * p.v_sn + lc4) * 4);
  }
  const int64_t kspan = ((int64_t)(kend - 1) * p.k_sn + HD) * 4;
  const int64_t vspan = ((int64_t)(kend - 1) * p.v_sn + HD) * 4;
  auto load_kv = [&](int kbase) {
    const int64_t ko = (int64_t)kbase * p.k_sn, vo = (int64_t)kbase * p.v_sn;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kb + ko), (short)0, (int)(kspan - 4 * ko), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(vb + vo), (short)0, (int)(vspan - 4 * vo), 0x00020000);
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      rk[i] = __builtin_bit_cast(fx4, __builtin_amdgcn_raw_buffer_load_b128(krs, kvo[i], 0, 0));
      rv[i] = __builtin_bit_cast(fx4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vvo[i], 0, 0));
    }
  };

  load_kv(kbeg);
  for (int kbase = kbeg; kbase < kend; kbase += KTT) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      *(fx4*)&Ks[lrow + 4 * NW * i][lc4] = rk[i];
      *(fx4*)&Vs[lrow + 4 * NW * i][lc4] = rv[i];
    }
    __syncthreads();
    if (kbase + KTT < kend) load_kv(kbase + KTT);

#pragma unroll
    for (int sub = 0; sub < KTT / 32; ++sub) {
      const int sb = kbase + sub * 32;
      if (sb >= kend) break;
      // S^T block: A = K rows (key l32, k = 32*hl + t), B = Q^T.
      floatx16 s = {};
      const float* kr = &Ks[sub * 32 + l32][hl * 32];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const fx4 kf = *(const fx4*)(kr + 4 * t);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qf[4 * t + 0], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qf[4 * t + 1], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qf[4 * t + 2], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qf[4 * t + 3], s, 0, 0, 0);
      }
      if (sb + 32 > kend) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = sb + 8 * (r >> 2) + 4 * hl + (r & 3);
          if (key >= kend) s[r] = -INFINITY;
        }
      }
      float mb = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mb = fmaxf(mb, s[r]);
      mb = fmaxf(mb, __shfl_xor(mb, 32));
      // Lazy rescaling: the reference maximum m_run only moves (and O, l
      // are rescaled) when some query of the wave sees a score more than
      // 2^8 above it, so exp2(s - m_run) <= 256 and the rescale multiplies
      // are skipped for most blocks (the first block always moves it from
      // -inf). O / l is unchanged by the choice of reference.
      const float m_cand = fmaxf(m_run, mb);
      if (__any(m_cand > m_run + 8.0f)) {
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_cand);
        l_run *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          o0[r] *= alpha;
          o1[r] *= alpha;
        }
        m_run = m_cand;
      }
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(s[r] - m_run);
        ps += s[r];
      }
      l_run += ps;
      // O^T += V^T P^T: A = V^T (hd row l32, k = key of register st).
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int kr2 = sub * 32 + 8 * (st >> 2) + 4 * hl + (st & 3);
        const float v0 = Vs[kr2][l32];
        const float v1 = Vs[kr2][32 + l32];
        o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0, s[st], o0, 0, 0, 0);
        o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1, s[st], o1, 0, 0, 0);
      }
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const int q = q0 + l32;
  if (SPLIT) {
    if (q < Nq) {
      const int64_t slot =
          (((int64_t)(grp * Bcount + b) * p.H + head) * Nq + q) * ns + krange;
      float* po = batch.part_ws + slot * 64;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        *(fx4*)(po + 8 * g + 4 * hl) = mk4(o0[4 * g], o0[4 * g + 1], o0[4 * g + 2], o0[4 * g + 3]);
        *(fx4*)(po + 32 + 8 * g + 4 * hl) =
            mk4(o1[4 * g], o1[4 * g + 1], o1[4 * g + 2], o1[4 * g + 3]);
      }
      if (hl == 0) {
        float* pml = batch.part_ws + batch.part_ws_elems - 2 * (slot + 1);
        pml[0] = m_run;
        pml[1] = l_tot;
      }
    }
    return;
  }
  const float inv = 1.0f / l_tot;
  if (q < Nq) {
    float* orow = ob + (int64_t)q * p.o_sn;
    // O^T layout: lane holds hd 8*g + 4*hl + {0..3} (+32 for o1) of query l32.
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      *(fx4*)(orow + 8 * g + 4 * hl) =
          mk4(o0[4 * g] * inv, o0[4 * g + 1] * inv, o0[4 * g + 2] * inv,
                      o0[4 * g + 3] * inv);
      *(fx4*)(orow + 32 + 8 * g + 4 * hl) =
          mk4(o1[4 * g] * inv, o1[4 * g + 1] * inv, o1[4 * g + 2] * inv,
                      o1[4 * g + 3] * inv);
    }
  }
}


// Merge of the key ranges of one (image, head, query): with M = max of the
// ranges' running maxima (base 2), O = sum_r O_r 2^(m_r - M) and
// l = sum_r l_r 2^(m_r - M) in range order, out = O / l. One thread per 4
// output dims.
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnBatch batch, int32_t Bcount) {
  const AttnArgs& p0 = batch.g[0];
  const int ns = batch.kv_split, H = p0.H, Nq = p0.Nq;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)batch.ngroups * Bcount * H * Nq * 16;
  if (i >= total) return;
  const int d4 = (int)(i & 15) * 4;
  const int64_t uq = i >> 4;  // (unit, query)
  const int q = (int)(uq % Nq);
  const int64_t u = uq / Nq;
  const int head = (int)(u % H);
  const int gb = (int)(u / H);
  const int grp = gb / Bcount, b = gb - grp * Bcount;
  const AttnArgs& p = batch.g[grp];
  const float* pml_end = batch.part_ws + batch.part_ws_elems;
  float mmax = -INFINITY;
  for (int r = 0; r < ns; ++r) mmax = fmaxf(mmax, pml_end[-2 * (uq * ns + r + 1)]);
  float l = 0.f;
  fx4 o = mk4(0.f, 0.f, 0.f, 0.f);
  for (int r = 0; r < ns; ++r) {
    const int64_t slot = uq * ns + r;
    const float w = exp2f(pml_end[-2 * (slot + 1)] - mmax);
    l = l + pml_end[-2 * (slot + 1) + 1] * w;
    const fx4 v = *(const fx4*)(batch.part_ws + slot * 64 + d4);
    o = mk4(o.x + v.x * w, o.y + v.y * w, o.z + v.z * w, o.w + v.w * w);
  }
  const float inv = 1.0f / l;
  *(fx4*)(p.o + (int64_t)b * p.o_sb + (int64_t)head * p.o_sh + (int64_t)q * p.o_sn + d4) =
      mk4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
}

// bf16-input / fp32-accumulate variant (v_mfma_f32_32x32x16_bf16), softmax in
// fp32. Q, K and V are read in fp32 and rounded to bf16 (nearest even).
//   S^T = K . Q^T: MFMA slice t (hd 16t .. 16t+15) takes, for lane half h,
//     hd 16t + 8h .. +7 of the lane's key row (A) and query (B).
//   O^T += V^T . P^T: slice s of a 32-key block takes, for lane half h, keys
//     {16s + 4h + 0..3, 16s + 8 + 4h + 0..3} -- exactly the keys the lane
//     holds in S^T accumulator registers 8s .. 8s+7 -- so P is converted in
//     registers; V is staged transposed in LDS (hd-major) so a lane reads
//     its 2 x 4 keys with two 8-byte loads.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Transposed V tile of the bf16 kernel: hd row h holds its 64 keys as 16
// groups of 4 (8 bytes each) in unpadded 128-byte rows, key group G in slot
// G ^ vt_swz(h). On gfx950 LDS writes resolve 32 banks (16 lanes of 8 bytes
// per cycle) and reads 64 banks (32 lanes of 8 bytes per cycle); with this
// slot order the transposing writes (16 lanes: rows 4c + j, c < 16, one key
// group) and the MFMA operand reads (32 lanes: rows l, l < 32, one key group)
// each touch distinct banks. The rows of 72 keys used before cost 8 cycles
// per write cycle (an 8-way conflict) and 2 per read.
__device__ __forceinline__ int vt_swz(int h) { return ((h >> 2) ^ (((h >> 1) & 1) << 3)) & 15; }

// INH: q, k and v hold bf16 (written so by the projection GEMMs); their K and V
// tiles go to LDS without conversion and the loads move half the bytes.
template <bool INH>
__global__ __launch_bounds__(256, 2) void attn_fwd_bf16_kernel(AttnBatch batch, int32_t Bcount) {
  const AttnTile tile = attn_tile();
  const int grp = tile.z / Bcount;
  const int b = tile.z - grp * Bcount;
  const AttnArgs& p = batch.g[grp];
  const int head = tile.y;
  const int Nq = p.Nq, Nkv = p.Nkv;

  __shared__ __attribute__((aligned(16))) __bf16 Ks[KT][HD + 8];
  __shared__ __attribute__((aligned(16))) __bf16 Vt[HD * KT];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  // element offsets of the lane's V^T operand reads, [row half e][sub][sl][u]
  // for hd row 32 e + l32 and key group 8 sub + 4 sl + 2 u + hl
  int vto[2][8];
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int ix = 0; ix < 8; ++ix) {
      const int h = 32 * e + l32, G = 2 * ix + hl;
      vto[e][ix] = h * KT + 4 * (G ^ vt_swz(h));
    }

  // element type of q, k, v: fp32, or bf16 (INH); strides are in elements
  typedef typename std::conditional<INH, __bf16, float>::type in_t;
  constexpr int ES = sizeof(in_t);
  const in_t* qb = (const in_t*)p.q + (int64_t)b * p.q_sb + (int64_t)head * p.q_sh;
  const in_t* kb = (const in_t*)p.k + (int64_t)b * p.k_sb + (int64_t)head * p.k_sh;
  const in_t* vb = (const in_t*)p.v + (int64_t)b * p.v_sb + (int64_t)head * p.v_sh;
  float* ob = p.o + (int64_t)b * p.o_sb + (int64_t)head * p.o_sh;

  const int q0 = tile.x * QT + wave * 32;
  const float qscale = p.scale * 1.4426950408889634f;
  bf16x8 qf[4];
  {
    const int qrow = min(q0 + l32, Nq - 1);
    const in_t* qr = qb + (int64_t)qrow * p.q_sn + hl * 8;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      fx4 v0, v1;
      if constexpr (INH) {
        const u32x4 w = *(const u32x4*)(qr + 16 * t);
        v0 = mk4(bf16_lo(w[0]), bf16_hi(w[0]), bf16_lo(w[1]), bf16_hi(w[1]));
        v1 = mk4(bf16_lo(w[2]), bf16_hi(w[2]), bf16_lo(w[3]), bf16_hi(w[3]));
      } else {
        v0 = *(const fx4*)(qr + 16 * t);
        v1 = *(const fx4*)(qr + 16 * t + 4);
      }
      const u32x4 h = {cvt_pk_bf16(v0.x * qscale, v0.y * qscale),
                       cvt_pk_bf16(v0.z * qscale, v0.w * qscale),
                       cvt_pk_bf16(v1.x * qscale, v1.y * qscale),
                       cvt_pk_bf16(v1.z * qscale, v1.w * qscale)};
      qf[t] = __builtin_bit_cast(bf16x8, h);
    }
  }

  floatx16 o0 = {}, o1 = {};
  float m_run = -INFINITY, l_run = 0.f;
  // rank-one operands of the reference subtraction: k slots 0 and 1 of the
  // lanes with hl == 0 hold 1 (key side) and the two bf16 terms -m_hi, -m_lo
  // of -m_run (query side)
  bf16x8 ones_k0 = {}, negm_k0 = {};
  ones_k0[0] = hl == 0 ? (__bf16)1.0f : (__bf16)0.0f;
  ones_k0[1] = ones_k0[0];

  const int lrow = tid >> 4, lc4 = (tid & 15) * 4;
  fx4 rk[4], rv[4];     // fp32 inputs: 4 values each
  uint64_t hk[4], hv[4];  // bf16 inputs (INH): 4 values each
  // K rows lrow + 16 i; V rows 4 lrow + i, so each thread holds four
  // consecutive keys of V and writes its transpose with 8-byte stores.
  // The loads go through buffer resources whose base is the tile's first key
  // row (scalar registers) and whose size ends at the last key's 64 values:
  // the lane offsets stay fixed across tiles, and rows at or past Nkv are out
  // of range and read as zero (rows are at least HD apart, checked on the
  // host). The whole (image, head) span is below 2^31 bytes (host check).
  uint32_t kvo[4], vvo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kvo[i] = (uint32_t)(((int64_t)(lrow + 16 * i) * p.k_sn + lc4) * ES);
    vvo[i] = (uint32_t)(((int64_t)(4 * lrow + i) * p.v_sn + lc4) * ES);
  }
  const int64_t kspan = ((int64_t)(Nkv - 1) * p.k_sn + HD) * ES;
  const int64_t vspan = ((int64_t)(Nkv - 1) * p.v_sn + HD) * ES;
#define GS_ATT_LOAD(KB)                                                                      \
  {                                                                                          \
    const int64_t ko = (int64_t)(KB) * p.k_sn, vo = (int64_t)(KB) * p.v_sn;                  \
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(                    \
        (void*)(kb + ko), (short)0, (int)(kspan - ES * ko), 0x00020000);                     \
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(                    \
        (void*)(vb + vo), (short)0, (int)(vspan - ES * vo), 0x00020000);                     \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                          \
      if constexpr (INH) {                                                                   \
        hk[i] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(krs, kvo[i], 0, 0)); \
        hv[i] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(vrs, vvo[i], 0, 0)); \
      } else {                                                                               \
        rk[i] = __builtin_bit_cast(fx4, __builtin_amdgcn_raw_buffer_load_b128(krs, kvo[i], 0, 0)); \
        rv[i] = __builtin_bit_cast(fx4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vvo[i], 0, 0)); \
      }                                                                                      \
    }                                                                                        \
  }

  GS_ATT_LOAD(0)
  for (int kbase = 0; kbase < Nkv; kbase += KT) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (INH) {
        *(uint64_t*)&Ks[lrow + 16 * i][lc4] = hk[i];
        // V^T: column lc4 + i of the keys 4 lrow .. + 3, the 16-bit value i
        // of each of the four rows, packed in key order
        const int sh = 16 * (i & 1), w = i >> 1;
        uint32_t e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = (uint32_t)(hv[j] >> (32 * w + sh)) & 0xffffu;
        *(uint64_t*)&Vt[(lc4 + i) * KT + 4 * (lrow ^ vt_swz(lc4 + i))] =
            (uint64_t)(e[0] | (e[1] << 16)) | ((uint64_t)(e[2] | (e[3] << 16)) << 32);
      } else {
        *(uint64_t*)&Ks[lrow + 16 * i][lc4] =
            (uint64_t)cvt_pk_bf16(rk[i].x, rk[i].y) | ((uint64_t)cvt_pk_bf16(rk[i].z, rk[i].w) << 32);
        // V^T (head-dim major): column lc4 + i of the keys 4 lrow .. 4 lrow + 3
        const float c0[4] = {rv[0].x, rv[0].y, rv[0].z, rv[0].w};
        const float c1[4] = {rv[1].x, rv[1].y, rv[1].z, rv[1].w};
        const float c2[4] = {rv[2].x, rv[2].y, rv[2].z, rv[2].w};
        const float c3[4] = {rv[3].x, rv[3].y, rv[3].z, rv[3].w};
        *(uint64_t*)&Vt[(lc4 + i) * KT + 4 * (lrow ^ vt_swz(lc4 + i))] =
            (uint64_t)cvt_pk_bf16(c0[i], c1[i]) | ((uint64_t)cvt_pk_bf16(c2[i], c3[i]) << 32);
      }
    }
    __syncthreads();
    GS_ATT_LOAD(min(kbase + KT, ((Nkv - 1) / KT) * KT))

#pragma unroll
    for (int sub = 0; sub < KT / 32; ++sub) {
      const int sb = kbase + sub * 32;
      if (sb >= Nkv) break;
      // Scores relative to the running reference m_run = m_hi + m_lo, a sum
      // of two bf16 values: a fifth MFMA adds the rank-one product
      // ones x (-m_hi, -m_lo) (k slots 0 and 1 of the halves with hl == 0),
      // so the exponentials take the accumulators as they are and the VALU,
      // which bounds this kernel, does no subtraction. Two terms keep m_run
      // within 2^-16 of the running maximum at any magnitude (one bf16 term
      // would miss it by up to half a bf16 ulp: 128 at |m| = 2^15, enough to
      // overflow exp2).
      floatx16 s = {};
      const __bf16* kr = &Ks[sub * 32 + l32][hl * 8];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8*)(kr + 16 * t), qf[t], s, 0, 0,
                                                    0);
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ones_k0, negm_k0, s, 0, 0, 0);
      if (sb + 32 > Nkv) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = sb + 8 * (r >> 2) + 4 * hl + (r & 3);
          if (key >= Nkv) s[r] = -INFINITY;
        }
      }
      float mb = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mb = fmaxf(mb, s[r]);
      mb = fmaxf(mb, __shfl_xor(mb, 32));  // block maximum relative to m_run (0 at first)
      // Lazy rescaling: the reference maximum m_run only moves (and O, l
      // are rescaled) when some query of the wave sees a score more than
      // 2^8 above it, so exp2(s - m_run) <= 2^8 (to m_run's 2^-16 relative
      // residual) and the rescale multiplies are skipped for most blocks (the first block
      // always moves it from -inf). O / l is unchanged by the choice of
      // reference.
      if (__any(m_run == -INFINITY || mb > 8.0f)) {
        const float m_base = m_run == -INFINITY ? 0.f : m_run;
        const float m_t = fmaxf(m_run, m_base + mb);
        const __bf16 m_hi = (__bf16)m_t;
        const __bf16 m_lo = (__bf16)(m_t - (float)m_hi);
        const float m_new = (float)m_hi + (float)m_lo;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          o0[r] *= alpha;
          o1[r] *= alpha;
        }
        const float shift = m_new - m_base;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] -= shift;
        m_run = m_new;
        negm_k0[0] = hl == 0 ? -m_hi : (__bf16)0.0f;
        negm_k0[1] = hl == 0 ? -m_lo : (__bf16)0.0f;
      }
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(s[r]);
        ps += s[r];
      }
      l_run += ps;
      // P in bf16, the PV product's B operand
      u32x4 pq[2];
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int u = 0; u < 4; ++u) pq[sl][u] = cvt_pk_bf16(s[8 * sl + 2 * u], s[8 * sl + 2 * u + 1]);
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        const bf16x8 pb = __builtin_bit_cast(bf16x8, pq[sl]);
        // keys sub*32 + 16 sl + 4 hl + {0..3, 8..11}: key groups 8 sub + 4 sl + hl (+2)
        const int ix = 4 * sub + 2 * sl;
        const bf16x4 va0 = *(const bf16x4*)&Vt[vto[0][ix]];
        const bf16x4 va1 = *(const bf16x4*)&Vt[vto[0][ix + 1]];
        const bf16x4 vb0 = *(const bf16x4*)&Vt[vto[1][ix]];
        const bf16x4 vb1 = *(const bf16x4*)&Vt[vto[1][ix + 1]];
        const bf16x8 v0 = {va0.x, va0.y, va0.z, va0.w, va1.x, va1.y, va1.z, va1.w};
        const bf16x8 v1 = {vb0.x, vb0.y, vb0.z, vb0.w, vb1.x, vb1.y, vb1.z, vb1.w};
        o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v0, pb, o0, 0, 0, 0);
        o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v1, pb, o1, 0, 0, 0);
      }
    }
  }
#undef GS_ATT_LOAD

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  const int q = q0 + l32;
  if (q < Nq && p.o_bf16) {  // bf16 output for a bf16-input projection
    __bf16* orow = (__bf16*)p.o + (int64_t)b * p.o_sb + (int64_t)head * p.o_sh + (int64_t)q * p.o_sn;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const bf16x4 h0 = {(__bf16)(o0[4 * g] * inv), (__bf16)(o0[4 * g + 1] * inv),
                         (__bf16)(o0[4 * g + 2] * inv), (__bf16)(o0[4 * g + 3] * inv)};
      const bf16x4 h1 = {(__bf16)(o1[4 * g] * inv), (__bf16)(o1[4 * g + 1] * inv),
                         (__bf16)(o1[4 * g + 2] * inv), (__bf16)(o1[4 * g + 3] * inv)};
      *(bf16x4*)(orow + 8 * g + 4 * hl) = h0;
      *(bf16x4*)(orow + 32 + 8 * g + 4 * hl) = h1;
    }
  } else if (q < Nq) {
    float* orow = ob + (int64_t)q * p.o_sn;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      *(fx4*)(orow + 8 * g + 4 * hl) =
          mk4(o0[4 * g] * inv, o0[4 * g + 1] * inv, o0[4 * g + 2] * inv, o0[4 * g + 3] * inv);
      *(fx4*)(orow + 32 + 8 * g + 4 * hl) =
          mk4(o1[4 * g] * inv, o1[4 * g + 1] * inv, o1[4 * g + 2] * inv, o1[4 * g + 3] * inv);
    }
  }
}

// fp32 attention through bf16 matrix cores ("bf16x6", precision 2): the
// operands of both products (Q and K for the scores, P and V for the output)
// are split exactly into three bf16 terms x = x0 + x1 + x2 and each product
// is accumulated in fp32 from the six term products of relative size
// >= 2^-16 (the same scheme as gemm_x6_kernel; fp32-level accuracy). Layout
// and softmax as attn_fwd_bf16_kernel; the K / V tiles are stored as three
// bf16 planes each (55 KB of LDS), Q's planes stay in registers.
__device__ __forceinline__ void split3_8(const float* v, bf16x8& h, bf16x8& m, bf16x8& l) {
  u32x4 ph, pm, pl;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t a, b, c;
    split3_pk(v[2 * i], v[2 * i + 1], a, b, c);
    ph[i] = a;
    pm[i] = b;
    pl[i] = c;
  }
  h = __builtin_bit_cast(bf16x8, ph);
  m = __builtin_bit_cast(bf16x8, pm);
  l = __builtin_bit_cast(bf16x8, pl);
}

__global__ __launch_bounds__(256, 2) void attn_fwd_x6_kernel(AttnBatch batch, int32_t Bcount) {
  const AttnTile tile = attn_tile();
  const int grp = tile.z / Bcount;
  const int b = tile.z - grp * Bcount;
  const AttnArgs& p = batch.g[grp];
  const int head = tile.y;
  const int Nq = p.Nq, Nkv = p.Nkv;

  __shared__ __attribute__((aligned(16))) __bf16 Ks[3][KT][HD + 8];
  __shared__ __attribute__((aligned(16))) __bf16 Vt[3][HD][KT + 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;

  const float* qb = p.q + (int64_t)b * p.q_sb + (int64_t)head * p.q_sh;
  const float* kb = p.k + (int64_t)b * p.k_sb + (int64_t)head * p.k_sh;
  const float* vb = p.v + (int64_t)b * p.v_sb + (int64_t)head * p.v_sh;
  float* ob = p.o + (int64_t)b * p.o_sb + (int64_t)head * p.o_sh;

  const int q0 = tile.x * QT + wave * 32;
  const float qscale = p.scale * 1.4426950408889634f;
  bf16x8 qf[3][4];  // [term][16-wide head-dim slice], scaled as the fp32 kernel
  {
    const int qrow = min(q0 + l32, Nq - 1);
    const float* qr = qb + (int64_t)qrow * p.q_sn + hl * 8;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const fx4 v0 = *(const fx4*)(qr + 16 * t);
      const fx4 v1 = *(const fx4*)(qr + 16 * t + 4);
      const float v[8] = {v0.x * qscale, v0.y * qscale, v0.z * qscale, v0.w * qscale,
                          v1.x * qscale, v1.y * qscale, v1.z * qscale, v1.w * qscale};
      split3_8(v, qf[0][t], qf[1][t], qf[2][t]);
    }
  }

  floatx16 o0 = {}, o1 = {};
  float m_run = -INFINITY, l_run = 0.f;

  const int lrow = tid >> 4, lc4 = (tid & 15) * 4;
  fx4 rk[4], rv[4];
  // K rows lrow + 16 i; V rows 4 lrow + i, so each thread holds four
  // consecutive keys of V and writes its transpose with 8-byte stores. The
  // loads go through buffer resources based at the tile's first key row and
  // ending at the last key's 64 values (as in attn_fwd_kernel): fixed lane
  // offsets, rows at or past Nkv read as zero.
  uint32_t kvo[4], vvo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kvo[i] = (uint32_t)(((int64_t)(lrow + 16 * i) * p.k_sn + lc4) * 4);
    vvo[i] = (uint32_t)(((int64_t)(4 * lrow + i) * p.v_sn + lc4) * 4);
  }
  const int64_t kspan = ((int64_t)(Nkv - 1) * p.k_sn + HD) * 4;
  const int64_t vspan = ((int64_t)(Nkv - 1) * p.v_sn + HD) * 4;
#define GS_ATT_LOAD(KB)                                                                      \
  {                                                                                          \
    const int64_t ko = (int64_t)(KB) * p.k_sn, vo = (int64_t)(KB) * p.v_sn;                  \
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(                    \
        (void*)(kb + ko), (short)0, (int)(kspan - 4 * ko), 0x00020000);                      \
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(                    \
        (void*)(vb + vo), (short)0, (int)(vspan - 4 * vo), 0x00020000);                      \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                          \
      rk[i] = __builtin_bit_cast(fx4, __builtin_amdgcn_raw_buffer_load_b128(krs, kvo[i], 0, 0)); \
      rv[i] = __builtin_bit_cast(fx4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vvo[i], 0, 0)); \
    }                                                                                        \
  }
// product of the three-term operands A[ta] x B[tb], smallest terms first
#define GS_X6_MM(ACC, A, B)                                                           \
  ACC = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[2], B[0], ACC, 0, 0, 0);           \
  ACC = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[0], B[2], ACC, 0, 0, 0);           \
  ACC = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[1], B[1], ACC, 0, 0, 0);           \
  ACC = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[1], B[0], ACC, 0, 0, 0);           \
  ACC = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[0], B[1], ACC, 0, 0, 0);           \
  ACC = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[0], B[0], ACC, 0, 0, 0);

  GS_ATT_LOAD(0)
  for (int kbase = 0; kbase < Nkv; kbase += KT) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = lrow + 16 * i;
      uint32_t k0[3], k1[3];
      split3_pk(rk[i].x, rk[i].y, k0[0], k0[1], k0[2]);
      split3_pk(rk[i].z, rk[i].w, k1[0], k1[1], k1[2]);
#pragma unroll
      for (int u = 0; u < 3; ++u)
        *(uint64_t*)&Ks[u][key][lc4] = (uint64_t)k0[u] | ((uint64_t)k1[u] << 32);
      // V^T (head-dim major): column lc4 + i of the keys 4 lrow .. 4 lrow + 3
      const float c0[4] = {rv[0].x, rv[0].y, rv[0].z, rv[0].w};
      const float c1[4] = {rv[1].x, rv[1].y, rv[1].z, rv[1].w};
      const float c2[4] = {rv[2].x, rv[2].y, rv[2].z, rv[2].w};
      const float c3[4] = {rv[3].x, rv[3].y, rv[3].z, rv[3].w};
      uint32_t v0[3], v1[3];
      split3_pk(c0[i], c1[i], v0[0], v0[1], v0[2]);
      split3_pk(c2[i], c3[i], v1[0], v1[1], v1[2]);
#pragma unroll
      for (int u = 0; u < 3; ++u)
        *(uint64_t*)&Vt[u][lc4 + i][4 * lrow] = (uint64_t)v0[u] | ((uint64_t)v1[u] << 32);
    }
    __syncthreads();
    GS_ATT_LOAD(min(kbase + KT, ((Nkv - 1) / KT) * KT))

#pragma unroll
    for (int sub = 0; sub < KT / 32; ++sub) {
      const int sb = kbase + sub * 32;
      if (sb >= Nkv) break;
      floatx16 s = {};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bf16x8 kf[3];
#pragma unroll
        for (int u = 0; u < 3; ++u) kf[u] = *(const bf16x8*)&Ks[u][sub * 32 + l32][hl * 8 + 16 * t];
        const bf16x8 qt[3] = {qf[0][t], qf[1][t], qf[2][t]};
        GS_X6_MM(s, kf, qt)
      }
      if (sb + 32 > Nkv) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = sb + 8 * (r >> 2) + 4 * hl + (r & 3);
          if (key >= Nkv) s[r] = -INFINITY;
        }
      }
      float mb = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mb = fmaxf(mb, s[r]);
      mb = fmaxf(mb, __shfl_xor(mb, 32));
      // lazy rescaling as in attn_fwd_kernel
      const float m_cand = fmaxf(m_run, mb);
      if (__any(m_cand > m_run + 8.0f)) {
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_cand);
        l_run *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          o0[r] *= alpha;
          o1[r] *= alpha;
        }
        m_run = m_cand;
      }
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(s[r] - m_run);
        ps += s[r];
      }
      l_run += ps;
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        float pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[i] = s[8 * sl + i];
        bf16x8 pb[3];
        split3_8(pv, pb[0], pb[1], pb[2]);
        const int k0 = sub * 32 + 16 * sl + 4 * hl;
        bf16x8 v0[3], v1[3];
#pragma unroll
        for (int u = 0; u < 3; ++u) {
          const bf16x4 va0 = *(const bf16x4*)&Vt[u][l32][k0];
          const bf16x4 va1 = *(const bf16x4*)&Vt[u][l32][k0 + 8];
          const bf16x4 vb0 = *(const bf16x4*)&Vt[u][32 + l32][k0];
          const bf16x4 vb1 = *(const bf16x4*)&Vt[u][32 + l32][k0 + 8];
          v0[u] = bf16x8{va0.x, va0.y, va0.z, va0.w, va1.x, va1.y, va1.z, va1.w};
          v1[u] = bf16x8{vb0.x, vb0.y, vb0.z, vb0.w, vb1.x, vb1.y, vb1.z, vb1.w};
        }
        GS_X6_MM(o0, v0, pb)
        GS_X6_MM(o1, v1, pb)
      }
    }
  }
#undef GS_X6_MM
#undef GS_ATT_LOAD

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  const int q = q0 + l32;
  if (q < Nq) {
    float* orow = ob + (int64_t)q * p.o_sn;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      *(fx4*)(orow + 8 * g + 4 * hl) =
          mk4(o0[4 * g] * inv, o0[4 * g + 1] * inv, o0[4 * g + 2] * inv, o0[4 * g + 3] * inv);
      *(fx4*)(orow + 32 + 8 * g + 4 * hl) =
          mk4(o1[4 * g] * inv, o1[4 * g + 1] * inv, o1[4 * g + 2] * inv, o1[4 * g + 3] * inv);
    }
  }
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

int64_t attention_split_elems(const AttnBatch& bt, int prec) {
  const AttnArgs& a0 = bt.g[0];
  if (prec == 1 || a0.B <= 0 || a0.H <= 0 || a0.Nq <= 0 || a0.Nkv < 2 * KT) return 0;
  const int64_t units = (int64_t)a0.H * a0.B * bt.ngroups;
  const int64_t qtiles = (a0.Nq + QT - 1) / QT;
  if (bt.kv_split == 0 && units * qtiles >= 3 * kAttnCUs) return 0;
  const int64_t ranges = (a0.Nkv + KT - 1) / KT;  // the most a split uses
  return units * a0.Nq * ranges * 66;
}

int launch_attention(const AttnBatch& bt, hipStream_t s, int prec) {
  const bool bf16 = prec == 1, x6 = prec == 2;
  GS_REQUIRE(bt.ngroups >= 1 && bt.ngroups <= kMaxGroups, "attention: bad group count");
  const AttnArgs& a0 = bt.g[0];
  for (int i = 0; i < bt.ngroups; ++i) {
    const AttnArgs& a = bt.g[i];
    GS_REQUIRE(a.B == a0.B && a.H == a0.H && a.Nq == a0.Nq && a.Nkv == a0.Nkv,
               "attention: grouped problems must share shapes");
    GS_REQUIRE(a.q && a.k && a.v && a.o, "attention: null operand");
    GS_REQUIRE(!a.o_bf16 || bf16, "attention: bf16 output needs the bf16 kernel");
    GS_REQUIRE(!a.in_bf16 || (bf16 && a.q_sb % 8 == 0 && a.q_sh % 8 == 0 && a.q_sn % 8 == 0),
               "attention: bf16 q / k / v need the bf16 kernel and q strides that are multiples "
               "of 8");
    GS_REQUIRE(a.in_bf16 == a0.in_bf16, "attention: grouped problems must share the input type");
    GS_REQUIRE(aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.o),
               "attention: operands must be 16-byte aligned");
    const int64_t st[12] = {a.q_sb, a.q_sh, a.q_sn, a.k_sb, a.k_sh, a.k_sn,
                            a.v_sb, a.v_sh, a.v_sn, a.o_sb, a.o_sh, a.o_sn};
    for (int j = 0; j < 12; ++j)
      GS_REQUIRE(st[j] % 4 == 0 && st[j] >= 0, "attention: strides must be multiples of 4");
    // the kernels' buffer-resource K / V loads (see the kernels)
    GS_REQUIRE(a.k_sn >= HD && a.v_sn >= HD, "attention: the MFMA kernels need key rows >= 64 apart");
    GS_REQUIRE(((int64_t)(a.Nkv - 1) * std::max(a.k_sn, a.v_sn) + HD) * 4 < ((int64_t)1 << 31),
               "attention: the MFMA kernels need each (image, head) K / V span below 2 GiB");
  }
  GS_REQUIRE(a0.B > 0 && a0.H > 0 && a0.Nq > 0 && a0.Nkv > 0, "attention: bad sizes");
  GS_REQUIRE((int64_t)a0.B * bt.ngroups <= 65535 && a0.H <= 65535, "attention: grid too large");
  // fp32 launches with fewer workgroups than three per CU may split the keys
  // into ranges of a multiple of 64 keys. The split minimises
  //   ceil(workgroups / CUs) * (64-key tiles per range) + 0.25 ns units Nq / 16384
  // (a CU's key tiles, plus the merge pass's round trip of the ranges' partial
  // outputs), which picks the fastest measured split of the one-image /
  // one-pair launches: 16 heads x 1 image 2 ranges (40.8 us; 4 ranges 42.6),
  // 16 heads x 2 images 4 (57.8; 3 ranges 70.2), 12 heads x 2 chains 3
  // (49.5; 4 ranges 57.2); unsplit they take 63.9, 64.7 and 63.5 us.
  AttnBatch b = bt;
  const int64_t units = (int64_t)a0.H * a0.B * bt.ngroups;
  const int qtiles = (a0.Nq + QT - 1) / QT;
  const int requested = bt.kv_split;
  b.kv_split = 1;
  auto fits = [&](int ns) { return units * a0.Nq * ns * 66 <= b.part_ws_elems; };
  if (!bf16 && b.part_ws && a0.Nkv >= 2 * KT && requested > 1) {
    for (int want = requested; want >= 2; --want) {
      const int chunk = ((a0.Nkv + want - 1) / want + KT - 1) / KT * KT;
      const int ns = (a0.Nkv + chunk - 1) / chunk;
      if (ns >= 2 && fits(ns)) {
        b.kv_split = ns;
        b.kv_chunk = chunk;
        break;
      }
    }
  } else if (!bf16 && b.part_ws && a0.Nkv >= 2 * KT && requested == 0 &&
             units * qtiles < 3 * kAttnCUs) {
    const int ktiles = (a0.Nkv + KT - 1) / KT;
    double best = (double)((units * qtiles + kAttnCUs - 1) / kAttnCUs) * ktiles;
    for (int per = ktiles - 1; per >= 1; --per) {  // key tiles per range
      const int ns = (ktiles + per - 1) / per;
      if (ns < 2 || !fits(ns)) continue;
      const double cost = (double)((units * qtiles * ns + kAttnCUs - 1) / kAttnCUs) * per +
                          0.25 * ns * (double)units * a0.Nq / 16384.0;
      if (cost < best) {
        best = cost;
        b.kv_split = ns;
        b.kv_chunk = per * KT;
      }
    }
  }
  dim3 grid(qtiles * b.kv_split, a0.H, a0.B * bt.ngroups), block(256);
  hipEvent_t ev = prof_start(s);
  if (bf16) {
    if (a0.in_bf16)
      hipLaunchKernelGGL(attn_fwd_bf16_kernel<true>, grid, block, 0, s, b, a0.B);
    else
      hipLaunchKernelGGL(attn_fwd_bf16_kernel<false>, grid, block, 0, s, b, a0.B);
  } else if (x6 && b.kv_split == 1) {
    hipLaunchKernelGGL(attn_fwd_x6_kernel, grid, block, 0, s, b, a0.B);
  } else if (b.kv_split > 1) {
    GS_REQUIRE(aligned16(b.part_ws) && b.part_ws_elems % 4 == 0,
               "attention: scratch must be 16-byte aligned");
    hipLaunchKernelGGL((attn_fwd_kernel<true>), grid, block, 0, s, b, a0.B);
    const int64_t items = units * a0.Nq * 16;
    hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s,
                       b, a0.B);
  } else {
    hipLaunchKernelGGL((attn_fwd_kernel<false>), grid, block, 0, s, b, a0.B);
  }
  GS_CHECK_HIP(hipGetLastError());
  if (ev) {
    const double units = (double)a0.B * a0.H * bt.ngroups;
    std::string nm = bf16 ? "attn_fwd_bf16_kernel"
                          : (x6 && b.kv_split == 1 ? "attn_fwd_x6_kernel" : "attn_fwd_kernel");
    if (prof_per_shape())
      nm += " B=" + std::to_string(a0.B) + " H=" + std::to_string(a0.H) + " Nq=" +
            std::to_string(a0.Nq) + " groups=" + std::to_string(bt.ngroups) +
            (b.kv_split > 1 ? " kvsplit=" + std::to_string(b.kv_split) : std::string());
    prof_stop(s, ev, nm.c_str(), units * 4.0 * a0.Nq * (double)a0.Nkv * 64.0,
              units * 64.0 *
                  ((a0.in_bf16 ? 2.0 : 4.0) * (a0.Nq + 2.0 * a0.Nkv) + (a0.o_bf16 ? 2.0 : 4.0) * a0.Nq));
  }
  return 0;
}

}  // namespace gs
