// Split-factor sweep for the small launches of one image / one pair: times
// gs::launch_gemm and gs::launch_attention with every requested split on
// synthetic operands (the data behind plan_ksplit and the attention key-split
// target). Build and run from the repository root:
//   hipcc -O2 -std=c++17 crystal-gausplat_amd/tune/split_sweep.cpp -o split_sweep \
//     -Lcrystal-gausplat_amd -lgsplat_hip -Wl,-rpath,$PWD/crystal-gausplat_amd && ./split_sweep
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <vector>
#include "../csrc/internal.h"
using namespace gs;
#define CK(x) do { hipError_t e = (x); if (e) { printf("HIP %s\n", hipGetErrorString(e)); exit(1);} } while (0)
static float* dalloc(size_t n, float v) {
  float* p; CK(hipMalloc(&p, n * 4));
  std::vector<float> h(n); for (size_t i = 0; i < n; ++i) h[i] = v * (float)((i * 2654435761u) % 1000) / 1000.f;
  CK(hipMemcpy(p, h.data(), n * 4, hipMemcpyHostToDevice)); return p;
}
int main() {
  const int64_t WS = (int64_t)16 << 20;
  float* ws = dalloc(WS, 0.f);
  float* A = dalloc((size_t)1536 * 4096, 1.f);
  float* Bw = dalloc((size_t)4096 * 4096, 0.02f);
  float* C = dalloc((size_t)1536 * 4096 * 2, 0.f);
  float* R = dalloc((size_t)1536 * 4096, 1.f);
  float* bias = dalloc(8192, 0.1f);
  float* rc = dalloc(512 * 16, 1.f); float* rs = dalloc(512 * 16, 0.f);
  struct Sh { int M, N, K, g, flags; const char* nm; };
  Sh shapes[] = {
    {768, 3072, 1024, 1, EPI_BIAS | EPI_ROPE, "c0 qkv"}, {768, 4096, 1024, 1, EPI_BIAS | EPI_GELU, "c0 fc1"},
    {768, 1024, 4096, 1, EPI_BIAS | EPI_RES1, "c0 fc2"}, {768, 1024, 1024, 1, EPI_BIAS | EPI_RES1, "c0 proj"},
    {1536, 3072, 1024, 1, EPI_BIAS | EPI_ROPE, "c2 qkv"}, {1536, 4096, 1024, 1, EPI_BIAS | EPI_GELU, "c2 fc1"},
    {1536, 1024, 4096, 1, EPI_BIAS | EPI_RES1, "c2 fc2"}, {1536, 1024, 1024, 1, EPI_BIAS | EPI_RES1, "c2 proj"},
    {768, 768, 768, 2, EPI_BIAS | EPI_RES1, "c2 dproj"}, {768, 768, 3072, 2, EPI_BIAS | EPI_RES1, "c2 dfc2"},
    {768, 3072, 768, 2, EPI_BIAS | EPI_GELU, "c2 dfc1"}, {768, 2304, 768, 2, EPI_BIAS | EPI_ROPE, "c2 dqkv"},
    {768, 1536, 768, 2, EPI_BIAS | EPI_ROPE, "c2 dkv"},
  };
  hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
  for (auto& sh : shapes) {
    printf("%-9s M=%d N=%d K=%d g=%d:", sh.nm, sh.M, sh.N, sh.K, sh.g);
    for (int S : {1, 2, 3, 4, 6, 8, 12, 16}) {
      if ((sh.K / 32) % S || (sh.K / 32) / S < 2) continue;
      if ((int64_t)S * sh.M * sh.N * sh.g > WS) continue;
      GemmBatch b;
      b.ngroups = sh.g;
      for (int gi = 0; gi < sh.g; ++gi) {
        GemmArgs a; memset(&a, 0, sizeof(a));
        a.A = A; a.lda = sh.K; a.B = Bw; a.ldb = sh.K; a.C = C + (size_t)gi * sh.M * sh.N; a.ldc = sh.N;
        a.bias = bias; a.R1 = R; a.ldr1 = sh.N; a.M = sh.M; a.N = sh.N; a.K = sh.K; a.flags = sh.flags;
        a.rope_cos = rc; a.rope_sin = rs; a.rope_ncols = (sh.flags & EPI_ROPE) ? (sh.N / 64) * 64 : 0;
        a.tok_per_img = 768; a.grid_w = 32;
        b.g[gi] = a;
      }
      b.part_ws = ws; b.part_ws_elems = WS; b.ksplit = S == 1 ? 0 : S;
      if (S == 1) b.part_ws = nullptr;
      for (int w = 0; w < 3; ++w) if (launch_gemm(b, A_PLAIN, B_NT, false, 0, false)) { printf(" err %s", last_error()); break; }
      CK(hipEventRecord(e0, 0));
      for (int r = 0; r < 20; ++r) launch_gemm(b, A_PLAIN, B_NT, false, 0, false);
      CK(hipEventRecord(e1, 0)); CK(hipEventSynchronize(e1));
      float ms; CK(hipEventElapsedTime(&ms, e0, e1));
      const double us = ms * 1000.0 / 20;
      printf("  S%d %.1fus(%.0fTF)", S, us, 2.0 * sh.M * sh.N * (double)sh.K * sh.g / us / 1e6);
    }
    printf("\n"); fflush(stdout);
  }
  // attention key splits
  float* q = dalloc((size_t)2 * 768 * 3 * 1024, 0.1f);
  float* o = dalloc((size_t)2 * 768 * 1024 * 2, 0.f);
  struct At { int B, H, g; const char* nm; } ats[] = {{1, 16, 1, "c0 attn"}, {2, 16, 1, "c2 enc attn"}, {1, 12, 2, "c2 dec attn"}};
  for (auto& at : ats) {
    printf("%-12s B=%d H=%d g=%d:", at.nm, at.B, at.H, at.g);
    for (int ns : {1, 2, 3, 4, 6, 8, 12}) {
      AttnBatch b; b.ngroups = at.g;
      for (int gi = 0; gi < at.g; ++gi) {
        const int D = at.H * 64;
        AttnArgs a; memset(&a, 0, sizeof(a));
        a.q = q; a.k = q + D; a.v = q + 2 * D; a.o = o + (size_t)gi * 768 * D * at.B;
        a.q_sb = a.k_sb = a.v_sb = (int64_t)768 * 3 * D; a.q_sh = a.k_sh = a.v_sh = 64; a.q_sn = a.k_sn = a.v_sn = 3 * D;
        a.o_sb = (int64_t)768 * D; a.o_sh = 64; a.o_sn = D; a.B = at.B; a.H = at.H; a.Nq = a.Nkv = 768; a.scale = 0.125f;
        b.g[gi] = a;
      }
      b.part_ws = ws; b.part_ws_elems = WS; b.kv_split = ns;
      for (int w = 0; w < 3; ++w) if (launch_attention(b, 0, false)) { printf(" err %s", last_error()); break; }
      CK(hipEventRecord(e0, 0));
      for (int r = 0; r < 20; ++r) launch_attention(b, 0, false);
      CK(hipEventRecord(e1, 0)); CK(hipEventSynchronize(e1));
      float ms; CK(hipEventElapsedTime(&ms, e0, e1));
      printf("  ns%d %.1fus", ns, ms * 1000.0 / 20);
    }
    printf("\n"); fflush(stdout);
  }
  return 0;
}
