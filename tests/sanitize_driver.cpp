// Drives every function of the CPU oracle (oracle/oracle.c) and the host generator
// (mtorch_amd/csrc/rng.cpp) over ragged, empty and edge-case shapes, with every buffer sized
// exactly, so that an AddressSanitizer / UndefinedBehaviorSanitizer build reports any access
// outside a buffer, any overflow or invalid shift.  Built and run by tests/test_sanitized_builds.py
// with -fsanitize=address,undefined -fno-sanitize-recover=all; exit status 0 means clean.
// It also checks that the product generator (rng.cpp) and the oracle's produce the same draws.
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../include/mthip.h"
#include "../oracle/oracle.h"

namespace {

int failures = 0;

void expect(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s\n", what);
    ++failures;
  }
}

std::vector<float> randf(orc_rng& r, int64_t n, double std = 1.0) {
  std::vector<float> v((size_t)n);
  if (n) orc_fill_normal_f32(&r, v.data(), n, 0.0, std);
  return v;
}

std::vector<uint16_t> randh(orc_rng& r, int64_t n, double std = 1.0) {
  std::vector<uint16_t> v((size_t)n);
  if (n) orc_fill_normal_f16(&r, v.data(), n, 0.0, std);
  return v;
}

// Exact-size buffer of n elements of a dtype (ORC_F16 / ORC_F32), filled from the generator.
struct Buf {
  std::vector<float> f;
  std::vector<uint16_t> h;
  int dt;
  Buf(orc_rng& r, int dt_, int64_t n, double std = 1.0) : dt(dt_) {
    if (dt == ORC_F16)
      h = randh(r, n, std);
    else
      f = randf(r, n, std);
  }
  Buf(int dt_, int64_t n) : dt(dt_) {
    if (dt == ORC_F16)
      h.assign((size_t)n, 0);
    else
      f.assign((size_t)n, 0.0f);
  }
  void* p() { return dt == ORC_F16 ? (void*)h.data() : (void*)f.data(); }
};

void conversions() {
  const float edge[] = {0.0f, -0.0f, 65504.0f, 65520.0f, -65520.0f, 5.96e-8f, 2.98e-8f, 1e-10f, INFINITY, -INFINITY,
                        NAN, 1.0f, -2.5f, 3.14159f};
  const int n = (int)(sizeof(edge) / sizeof(edge[0]));
  std::vector<uint16_t> h((size_t)n);
  std::vector<float> back((size_t)n);
  orc_f2h_array(edge, h.data(), n);
  orc_h2f_array(h.data(), back.data(), n);
  expect(h[2] == 0x7bff && h[3] == 0x7c00 && h[4] == 0xfc00, "f2h overflow boundary");
  expect(std::isnan(back[10]), "NaN survives the round trip");
  for (uint32_t b = 0; b < 65536; ++b) {
    const float v = orc_h2f((uint16_t)b);
    if (!std::isnan(v)) expect(orc_f2h(v) == (uint16_t)b, "h2f -> f2h round trip");
  }
  expect(orc_d2h(1.0) == 0x3c00, "d2h(1)");
  std::vector<uint16_t> hh((size_t)n);
  std::vector<float> ff((size_t)n);
  orc_cast_f32_to_f16(edge, hh.data(), n);
  orc_cast_f16_to_f32(hh.data(), ff.data(), n);
  expect(std::memcmp(hh.data(), h.data(), n * 2) == 0, "cast equals f2h");
}

void generators() {
  // the product's host generator against the oracle's, draw for draw
  void* g = mthip_generator_create(7);
  orc_rng r;
  orc_rng_seed(&r, 7);
  for (int64_t n : {0, 1, 5, 64, 7}) {
    std::vector<float> a((size_t)n), b((size_t)n);
    expect(mthip_rng_normal(g, MTHIP_F32, n ? a.data() : nullptr, n, 0.5, 2.0) == MTHIP_OK, "rng_normal f32");
    if (n) orc_fill_normal_f32(&r, b.data(), n, 0.5, 2.0);
    expect(a == b, "normal f32 draws equal the oracle's");
    std::vector<uint16_t> ah((size_t)n), bh((size_t)n);
    expect(mthip_rng_normal(g, MTHIP_F16, n ? ah.data() : nullptr, n, 0.0, 1.0) == MTHIP_OK, "rng_normal f16");
    if (n) orc_fill_normal_f16(&r, bh.data(), n, 0.0, 1.0);
    expect(ah == bh, "normal f16 draws equal the oracle's");
    expect(mthip_rng_uniform(g, MTHIP_F32, n ? a.data() : nullptr, n, -1.0, 3.0) == MTHIP_OK, "rng_uniform f32");
    if (n) orc_fill_uniform_f32(&r, b.data(), n, -1.0, 3.0);
    expect(a == b, "uniform f32 draws equal the oracle's");
    expect(mthip_rng_uniform(g, MTHIP_F16, n ? ah.data() : nullptr, n, -1.0, 3.0) == MTHIP_OK, "rng_uniform f16");
    if (n) orc_fill_uniform_f16(&r, bh.data(), n, -1.0, 3.0);
    expect(ah == bh, "uniform f16 draws equal the oracle's");
    std::vector<double> d((size_t)n);
    expect(mthip_rng_normal(g, MTHIP_F64, n ? d.data() : nullptr, n, 0.0, 1.0) == MTHIP_OK, "rng_normal f64");
    expect(mthip_rng_uniform(g, MTHIP_F64, n ? d.data() : nullptr, n, 0.0, 1.0) == MTHIP_OK, "rng_uniform f64");
    // the f64 draws above: n normals, then n uniforms
    for (int64_t i = 0; i < n; ++i) orc_rng_next_normal(&r);
    for (int64_t i = 0; i < n; ++i) orc_rng_uniform_open(&r);
  }
  uint64_t st = 0;
  int spare_flag = 0;
  double spare = 0.0;
  expect(mthip_generator_get_state(g, &st, &spare_flag, &spare) == MTHIP_OK, "get_state");
  expect(mthip_generator_set_state(g, st, spare_flag, spare) == MTHIP_OK, "set_state");
  expect(mthip_generator_seed(g, 3) == MTHIP_OK, "seed");
  expect(mthip_rng_normal(nullptr, MTHIP_F32, nullptr, 1, 0, 1) != MTHIP_OK, "null generator refused");
  expect(mthip_rng_normal(g, MTHIP_F32, nullptr, -1, 0, 1) != MTHIP_OK, "negative count refused");
  expect(mthip_rng_normal(g, 99, nullptr, 0, 0, 1) != MTHIP_OK, "unknown dtype refused");
  mthip_generator_destroy(g);
  double a = 0, b = 0;
  orc_rng_normal_pair(&r, &a, &b);
  (void)orc_rng_next_u64(&r);
}

void contractions(orc_rng& r) {
  for (int dt : {ORC_F32, ORC_F16}) {
    for (auto [M, N, K] : std::vector<std::array<int64_t, 3>>{{0, 3, 4}, {1, 1, 1}, {5, 7, 3}, {9, 13, 77}}) {
      Buf x(r, dt, M * K), w(r, dt, N * K), b(r, dt, N), y(dt, M * N);
      expect(orc_linear(dt, x.p(), w.p(), b.p(), y.p(), M, N, K) == 0, "linear");
      expect(orc_linear(dt, x.p(), w.p(), nullptr, y.p(), M, N, K) == 0, "linear without bias");
      Buf bb(r, dt, K * N), c(dt, M * N), in(r, dt, M * N);
      expect(orc_matmul(dt, x.p(), bb.p(), c.p(), 1, M, N, K, 0, 0) == 0, "matmul");
      expect(orc_addmm(dt, in.p(), x.p(), bb.p(), c.p(), M, N, K, 0.5, 2.0) == 0, "addmm");
      expect(orc_addmm(dt, in.p(), x.p(), bb.p(), c.p(), M, N, K, 0.0, 0.0) == 0, "addmm alpha 0");
      // batched with a broadcast right operand
      Buf xa(r, dt, 3 * M * K), cb(dt, 3 * M * N);
      expect(orc_matmul(dt, xa.p(), bb.p(), cb.p(), 3, M, N, K, M * K, 0) == 0, "batched matmul");
    }
  }
}

void convolutions(orc_rng& r) {
  struct Cfg {
    int64_t B, C, H, W, O, k, s, p, d, g;
  };
  const Cfg cfgs[] = {{2, 5, 9, 8, 7, 3, 1, 1, 1, 1}, {1, 6, 10, 7, 4, 3, 2, 1, 1, 1}, {2, 4, 9, 9, 6, 3, 1, 2, 2, 2},
                      {1, 8, 6, 5, 5, 1, 1, 0, 1, 1}, {1, 3, 4, 4, 3, 3, 1, 1, 1, 1}, {1, 12, 2, 3, 8, 3, 1, 0, 1, 1},
                      {0, 4, 5, 5, 4, 3, 1, 1, 1, 1}, {1, 6, 5, 5, 6, 3, 1, 1, 1, 6}};
  for (int dt : {ORC_F32, ORC_F16}) {
    for (const Cfg& c : cfgs) {
      const int64_t OH = orc_conv2d_out_size(c.H, c.k, c.s, c.p, c.d), OW = orc_conv2d_out_size(c.W, c.k, c.s, c.p, c.d);
      if (OH <= 0 || OW <= 0) continue;
      Buf x(r, dt, c.B * c.C * c.H * c.W), w(r, dt, c.O * (c.C / c.g) * c.k * c.k, 0.2), b(r, dt, c.O),
          y(dt, c.B * c.O * OH * OW);
      expect(orc_conv2d(dt, x.p(), w.p(), b.p(), y.p(), c.B, c.C, c.H, c.W, c.O, c.k, c.k, c.s, c.s, c.p, c.p, c.d,
                        c.d, c.g) == 0,
             "conv2d");
      expect(orc_conv2d(dt, x.p(), w.p(), nullptr, y.p(), c.B, c.C, c.H, c.W, c.O, c.k, c.k, c.s, c.s, c.p, c.p, c.d,
                        c.d, c.g) == 0,
             "conv2d without bias");
    }
  }
}

void attention(orc_rng& r) {
  for (int dt : {ORC_F32, ORC_F16}) {
    for (auto [P, Lq, Lk, E, Ev] :
         std::vector<std::array<int64_t, 5>>{{1, 1, 1, 1, 1}, {2, 7, 11, 12, 6}, {3, 5, 77, 40, 40}, {0, 3, 3, 4, 4}}) {
      Buf q(r, dt, P * Lq * E), k(r, dt, P * Lk * E), v(r, dt, P * Lk * Ev), o(dt, P * Lq * Ev);
      std::vector<uint8_t> bm((size_t)(P * Lq * Lk));
      for (size_t i = 0; i < bm.size(); ++i) bm[i] = (uint8_t)((i * 7 + 3) % 5 != 0);
      std::vector<float> am = randf(r, P * Lq * Lk, 2.0);
      for (int causal : {0, 1})
        for (int has_scale : {0, 1})
          for (double scale : {0.0, -0.125, 0.3}) {
            expect(orc_sdpa(dt, q.p(), k.p(), v.p(), o.p(), P, Lq, Lk, E, Ev, 0, nullptr, causal, has_scale, scale) == 0,
                   "sdpa");
            expect(orc_sdpa(dt, q.p(), k.p(), v.p(), o.p(), P, Lq, Lk, E, Ev, 1, bm.data(), causal, has_scale,
                            scale) == 0,
                   "sdpa bool mask");
            expect(orc_sdpa(dt, q.p(), k.p(), v.p(), o.p(), P, Lq, Lk, E, Ev, 2, am.data(), causal, has_scale,
                            scale) == 0,
                   "sdpa additive mask");
          }
    }
  }
}

void normalisations_and_pointwise(orc_rng& r) {
  for (int dt : {ORC_F32, ORC_F16}) {
    for (auto [B, C, inner, G] : std::vector<std::array<int64_t, 4>>{{2, 8, 30, 4}, {1, 40, 63, 8}, {3, 32, 5, 32},
                                                                      {0, 4, 4, 2}, {1, 6, 0, 3}}) {
      Buf x(r, dt, B * C * inner), w(r, dt, C), b(r, dt, C), y(dt, B * C * inner);
      expect(orc_group_norm(dt, x.p(), w.p(), b.p(), y.p(), B, C, inner, G, 1e-5) == 0, "group_norm");
      expect(orc_group_norm(dt, x.p(), nullptr, nullptr, y.p(), B, C, inner, G, 1e-5) == 0, "group_norm no affine");
    }
    for (auto [rows, N] : std::vector<std::array<int64_t, 2>>{{5, 320}, {1, 1}, {7, 77}, {0, 8}}) {
      Buf x(r, dt, rows * N, 3.0), w(r, dt, N), b(r, dt, N), y(dt, rows * N);
      expect(orc_layer_norm(dt, x.p(), w.p(), b.p(), y.p(), rows, N, 1e-5) == 0, "layer_norm");
      expect(orc_layer_norm(dt, x.p(), nullptr, nullptr, y.p(), rows, N, 1e-5) == 0, "layer_norm no affine");
      for (int rank : {1, 2, 3}) expect(orc_softmax_lastdim(dt, x.p(), y.p(), rows, N, rank) == 0, "softmax");
      for (int odt : {ORC_F32, ORC_F16}) {
        Buf z(odt, rows * N);
        expect(orc_softmax_generic(dt, x.p(), odt, z.p(), rows, N) == 0, "softmax generic");
      }
      for (int approx : {0, 1}) expect(orc_gelu(dt, x.p(), y.p(), rows * N, approx) == 0, "gelu");
      expect(orc_silu(dt, x.p(), y.p(), rows * N) == 0, "silu");
      for (int op : {0, 1, 2}) expect(orc_binary(dt, op, x.p(), w.p(), y.p(), std::min<int64_t>(rows * N, N)) == 0, "binary");
    }
  }
  expect(std::fabs(orc_fast_erf_float(0.5f) - (float)std::erf(0.5)) < 1e-6f, "fast erf");
  expect(std::isfinite(orc_gelu_unit_polynomial_float(0.25f)), "gelu polynomial");
}

}  // namespace

int main() {
  orc_rng r;
  orc_rng_seed(&r, 2024);
  conversions();
  generators();
  contractions(r);
  convolutions(r);
  attention(r);
  normalisations_and_pointwise(r);
  if (failures) {
    std::fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  std::printf("sanitized oracle and generator: clean\n");
  return 0;
}
