// Memory-safety driver for the CPU oracle (test infrastructure only): runs
// every oracle entry point on small inputs, including the two-view pair in
// both compositions, so that a build with -fsanitize=address,undefined
// (make -C oracle sanitize) reports any out-of-bounds access, use of
// uninitialised heap memory reachable by ASan, or undefined behaviour.
//
//   oracle/_san/check WEIGHTS.bin
//
// WEIGHTS.bin: u32 count, then per tensor u32 name length, name bytes,
// u64 float count, float32 data (written by tests/test_oracle_sanitize.py).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <string>
#include <vector>

#include "oracle.h"

static std::map<std::string, std::vector<float>> g_w;

static const float* weight(const char* name, void*) {
  auto it = g_w.find(name);
  if (it == g_w.end()) {
    fprintf(stderr, "missing weight %s\n", name);
    exit(3);
  }
  return it->second.data();
}

static std::vector<float> pattern(size_t n, float scale, unsigned salt) {
  std::vector<float> v(n);
  for (size_t i = 0; i < n; ++i) v[i] = scale * sinf(0.37f * (float)(i + 1) + 0.11f * (float)salt);
  return v;
}

static bool finite_all(const std::vector<float>& v) {
  for (float x : v)
    if (!isfinite(x)) return false;
  return true;
}

#define CHECK(c)                                                  \
  do {                                                            \
    if (!(c)) {                                                   \
      fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
      return 1;                                                   \
    }                                                             \
  } while (0)

int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: check WEIGHTS.bin\n");
    return 2;
  }
  FILE* f = fopen(argv[1], "rb");
  CHECK(f);
  uint32_t count = 0;
  CHECK(fread(&count, 4, 1, f) == 1);
  for (uint32_t i = 0; i < count; ++i) {
    uint32_t len = 0;
    CHECK(fread(&len, 4, 1, f) == 1 && len < 512);
    std::string name(len, ' ');
    CHECK(fread(&name[0], 1, len, f) == len);
    uint64_t n = 0;
    CHECK(fread(&n, 8, 1, f) == 1);
    std::vector<float> v(n);
    CHECK(fread(v.data(), 4, n, f) == n);
    g_w[name] = std::move(v);
  }
  fclose(f);
  orc_set_threads(2);

  // primitives, blocked and literal loops
  {
    const int M = 5, K = 7, N = 3;
    auto x = pattern(M * K, 1.f, 1), w = pattern(N * K, 0.5f, 2), b = pattern(N, 0.1f, 3);
    std::vector<float> y(M * N), y2(M * N);
    for (int layout = 0; layout < 2; ++layout) {
      orc_linear(x.data(), M, K, w.data(), b.data(), N, y.data(), layout);
      orc_linear_naive(x.data(), M, K, w.data(), b.data(), N, y2.data(), layout);
      CHECK(memcmp(y.data(), y2.data(), y.size() * 4) == 0);
    }
    std::vector<float> ln(M * K);
    auto g = pattern(K, 1.f, 4), be = pattern(K, 0.1f, 5);
    orc_layernorm(x.data(), M, K, g.data(), be.data(), 1e-6f, ln.data());
    orc_gelu(x.data(), M * K, ln.data());
    orc_relu(x.data(), M * K, ln.data());
    orc_add(x.data(), x.data(), M * K, ln.data());
    CHECK(finite_all(ln));
  }
  {
    const int B = 2, H = 2, Nq = 5, Nkv = 7, hd = 8;
    auto q = pattern(B * H * Nq * hd, 1.f, 6), k = pattern(B * H * Nkv * hd, 1.f, 7),
         v = pattern(B * H * Nkv * hd, 1.f, 8);
    std::vector<float> o(q.size()), o2(q.size());
    orc_sdpa(q.data(), k.data(), v.data(), o.data(), B, H, Nq, Nkv, hd, 0.35f);
    orc_sdpa_naive(q.data(), k.data(), v.data(), o2.data(), B, H, Nq, Nkv, hd, 0.35f);
    CHECK(memcmp(o.data(), o2.data(), o.size() * 4) == 0);
  }
  {
    std::vector<float> c(16 * 16), s(16 * 16);
    orc_rope_table(16, 64, 100.f, c.data(), s.data());
    auto t = pattern(2 * 6 * 128, 1.f, 9);
    orc_rope2d(t.data(), 2, 6, 2, 64, 3, 100.f);
    std::vector<float> r(t.size());
    orc_rope_ref_token(t.data(), r.data(), 2, 2, 3, 128, 2, 100.f);
    CHECK(finite_all(t) && finite_all(r));
  }
  {
    auto img = pattern(2 * 3 * 32 * 48, 1.f, 10);
    std::vector<float> pt(2 * 6 * 768);
    orc_unfold(img.data(), 2, 3, 32, 48, 16, pt.data());
    const int B = 1, H = 5, W = 7, Ci = 3, Co = 4;
    auto x = pattern(B * H * W * Ci, 1.f, 11), w = pattern(Co * Ci * 3 * 3, 0.3f, 12),
         b = pattern(Co, 0.1f, 13);
    for (int st = 1; st <= 2; ++st) {
      const int Ho = (H + 2 - 3) / st + 1, Wo = (W + 2 - 3) / st + 1;
      std::vector<float> y(B * Ho * Wo * Co), y2(y.size());
      orc_conv2d(x.data(), B, H, W, Ci, w.data(), b.data(), Co, 3, st, 1, y.data());
      orc_conv2d_naive(x.data(), B, H, W, Ci, w.data(), b.data(), Co, 3, st, 1, y2.data());
      CHECK(memcmp(y.data(), y2.data(), y.size() * 4) == 0);
    }
    auto wt = pattern(Ci * Co * 4 * 4, 0.3f, 14);
    std::vector<float> yt(B * H * 4 * W * 4 * Co), up(B * 2 * H * 2 * W * Ci);
    orc_conv_transpose(x.data(), B, H, W, Ci, wt.data(), b.data(), Co, 4, yt.data());
    orc_upsample2x(x.data(), B, H, W, Ci, up.data());
    auto fsh = pattern(2 * 6 * 256 * 2, 1.f, 15);
    std::vector<float> desc(2 * 2 * 16 * 3 * 16 * 2);
    orc_pixel_shuffle(fsh.data(), 2, 2, 3, 512, 16, 2, desc.data());
    CHECK(finite_all(yt) && finite_all(up) && finite_all(desc));
  }
  {
    auto fr = pattern(9 * 11 * 3, 0.5f, 16);
    std::vector<float> rs(20 * 17 * 3), pre(1 * 3 * 20 * 17);
    orc_resize_image(fr.data(), 9, 11, 3, 20, 17, rs.data());
    orc_preprocess_image(rs.data(), 1, 20, 17, pre.data());
    auto pts = pattern(100 * 3, 1.f, 17), conf = pattern(100, 1.f, 18);
    std::vector<float> op(300), oc(100);
    const int64_t k = orc_collect_points(pts.data(), conf.data(), 100, 0.f, op.data(), oc.data());
    CHECK(k > 0 && k < 100);
  }

  // composites on the tiny configuration of the tests (img 64x96, grid 4x6)
  orc_config cfg = {64, 96, 16, 128, 2, 2, 256, 128, 3, 2, 256, 64, {32, 64, 96, 128}, {0, 1, 2, 3},
                    32, 256, 24, 1e-6f, 100.f, 0, 1, 0};
  const int B = 2, N = 24, Hi = 64, Wi = 96;
  auto i1 = pattern(B * 3 * Hi * Wi, 1.f, 19), i2 = pattern(B * 3 * Hi * Wi, 1.f, 20);
  for (int naive = 0; naive < 2; ++naive) {
    orc_set_naive(naive);
    std::vector<float> p1(B * Hi * Wi * 3), c1(B * Hi * Wi), d1(B * Hi * Wi * 24), p2(p1.size()),
        c2(c1.size()), d2(d1.size());
    CHECK(orc_mastr_pair(&cfg, weight, nullptr, i1.data(), i2.data(), B, p1.data(), c1.data(),
                         d1.data(), p2.data(), c2.data(), d2.data()) == 0);
    CHECK(finite_all(p1) && finite_all(c2) && finite_all(d2));
    std::vector<float> e1(B * N * 128), e2(e1.size()), f1(B * N * 128), f2(f1.size());
    CHECK(orc_mastr_pair_taps(&cfg, weight, nullptr, i1.data(), i2.data(), B, e1.data(),
                              e2.data(), f1.data(), f2.data()) == 0);
    const float* hooks[4] = {e1.data(), f1.data(), f1.data(), f1.data()};
    CHECK(orc_dpt_head(&cfg, weight, nullptr, "downstream_head1", hooks, B, 4, 6, p1.data(),
                       c1.data()) == 0);
  }
  orc_set_naive(0);
  // the reference composition (own-view memory, stub heads on the patch grid)
  orc_config ref = cfg;
  ref.composite = 1;
  ref.rope_mode = 2;
  ref.ln_eps = 1e-5f;
  {
    std::vector<float> p1(B * N * 3), c1(B * N), p2(p1.size()), c2(c1.size());
    CHECK(orc_mastr_pair(&ref, weight, nullptr, i1.data(), i2.data(), B, p1.data(), c1.data(),
                         nullptr, p2.data(), c2.data(), nullptr) == 0);
    CHECK(finite_all(p1) && finite_all(c2));
  }
  {
    std::vector<float> x(B * N * 128);
    for (size_t i = 0; i < x.size(); ++i) x[i] = 0.01f * (float)(i % 97);
    CHECK(orc_encoder_block(&cfg, "enc_blocks.1", weight, nullptr, x.data(), B, 4, 6) == 0);
    std::vector<float> enc(B * N * 128);
    CHECK(orc_encoder(&cfg, weight, nullptr, i1.data(), B, enc.data()) == 0);
    CHECK(finite_all(x) && finite_all(enc));
    std::vector<float> mem(B * N * 128), desc(B * Hi * Wi * 24);
    for (size_t i = 0; i < mem.size(); ++i) mem[i] = 0.02f * (float)(i % 89) - 0.5f;
    CHECK(orc_decoder_block(&cfg, "dec_blocks2.2", weight, nullptr, x.data(), mem.data(), B, 4,
                            6) == 0);
    CHECK(orc_local_features(&cfg, weight, nullptr, "downstream_head2", enc.data(), x.data(), B,
                             4, 6, desc.data()) == 0);
    CHECK(finite_all(x) && finite_all(desc));
    // every planted composition mistake runs clean too
    for (int m = 1; m <= 5; ++m) {
      orc_set_mutation(m);
      std::vector<float> p1(B * Hi * Wi * 3), c1(B * Hi * Wi), d1(desc.size()), p2(p1.size()),
          c2(c1.size()), d2(desc.size());
      CHECK(orc_mastr_pair(&cfg, weight, nullptr, i1.data(), i2.data(), B, p1.data(), c1.data(),
                           d1.data(), p2.data(), c2.data(), d2.data()) == 0);
      CHECK(finite_all(d1) && finite_all(p2));
    }
    orc_set_mutation(0);
  }
  printf("OK\n");
  return 0;
}
