// GPU test of the C++ shim (ef::hip) used the way the reference's engine uses ef::kern: a decode
// step written like Transformer::forward (src/model.cpp:212-275) with the packed products,
// embedding lookup and argmax on the GPU through ef::hip, the FP32 glue from the CPU oracle, and
// host std::vector activations (the drop-in path with PCIe staging).  Checked against the oracle's
// own Transformer and Sampler.  Exit status 0 = all checks passed.
#include <cmath>
#include <cstdio>
#include <random>
#include <vector>

#include "ef_hip_kern.hpp"
extern "C" {
#include "efo.h"
}

using ef::QType;
using ef::WeightView;

namespace {

struct Dims {
  std::size_t D = 256, F = 512, H = 4, KV = 2, hd = 64, V = 512, L = 2;
};

std::vector<std::uint8_t> quantize(QType t, std::size_t rows, std::size_t cols, std::mt19937& g) {
  std::normal_distribution<float> nd(0.0f, 0.02f);
  uint64_t rb = 0;
  efo_row_bytes(static_cast<int>(t), cols, &rb);
  std::vector<std::uint8_t> out(rows * rb);
  std::vector<float> row(cols);
  for (std::size_t r = 0; r < rows; ++r) {
    for (auto& v : row) v = nd(g);
    efo_quantize_row(static_cast<int>(t), row.data(), cols, out.data() + r * rb, 1);
  }
  return out;
}

int fails = 0;
void check(bool ok, const char* what) {
  std::printf("  %-58s %s\n", what, ok ? "ok" : "FAIL");
  if (!ok) ++fails;
}

}  // namespace

int main() {
  if (!ef::hip::available()) {
    std::printf("no gfx950 device\n");
    return 2;
  }
  const Dims d;
  const std::size_t kvd = d.KV * d.hd;
  std::mt19937 g(123);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  // weights: Q4_0 layers with k_proj of layer 0 in Q8_0, Q8_0 lm_head, BF16 embedding
  struct Layer {
    std::vector<std::uint8_t> q, k, v, o, gate, up, down;
    std::vector<float> an, fn;
    QType kt = QType::Q4_0;
  };
  std::vector<Layer> layers(d.L);
  for (std::size_t l = 0; l < d.L; ++l) {
    Layer& w = layers[l];
    w.kt = l == 0 ? QType::Q8_0 : QType::Q4_0;
    w.q = quantize(QType::Q4_0, d.D, d.D, g);
    w.k = quantize(w.kt, kvd, d.D, g);
    w.v = quantize(QType::Q4_0, kvd, d.D, g);
    w.o = quantize(QType::Q4_0, d.D, d.D, g);
    w.gate = quantize(QType::Q4_0, d.F, d.D, g);
    w.up = quantize(QType::Q4_0, d.F, d.D, g);
    w.down = quantize(QType::Q4_0, d.D, d.F, g);
    w.an.resize(d.D);
    w.fn.resize(d.D);
    for (auto& v : w.an) v = 1.0f + 0.1f * nd(g);
    for (auto& v : w.fn) v = 1.0f + 0.1f * nd(g);
  }
  std::vector<std::uint8_t> embed = quantize(QType::BF16, d.V, d.D, g), lm = quantize(QType::Q8_0, d.V, d.D, g);
  std::vector<float> fnorm(d.D);
  for (auto& v : fnorm) v = 1.0f + 0.1f * nd(g);

  // the oracle's Transformer on the same bytes
  std::vector<efo_layer> ol(d.L);
  auto ow = [](QType t, const std::vector<std::uint8_t>& b, std::size_t r, std::size_t c) {
    return efo_weight{static_cast<int>(t), b.data(), r, c};
  };
  for (std::size_t l = 0; l < d.L; ++l) {
    const Layer& w = layers[l];
    ol[l] = efo_layer{ow(QType::Q4_0, w.q, d.D, d.D), ow(w.kt, w.k, kvd, d.D), ow(QType::Q4_0, w.v, kvd, d.D),
                      ow(QType::Q4_0, w.o, d.D, d.D), ow(QType::Q4_0, w.gate, d.F, d.D),
                      ow(QType::Q4_0, w.up, d.F, d.D), ow(QType::Q4_0, w.down, d.D, d.F), w.an.data(), w.fn.data()};
  }
  const efo_model om{{d.D, d.F, d.H, d.KV, d.hd, d.V, d.L, 64, 1e-5f, 10000.0f},
                     ow(QType::BF16, embed, d.V, d.D), ow(QType::Q8_0, lm, d.V, d.D), fnorm.data(), ol.data()};
  const std::vector<std::int32_t> ids = {1, 5, 9, 33, 2, 17, 17, 4};
  efo_transformer* ot = efo_transformer_create(&om, ids.size(), nullptr, EFO_BACKEND_AVX2);

  // the same step written like Transformer::forward, products through ef::hip
  std::vector<WeightView> wq(d.L), wk(d.L), wv(d.L), wo(d.L), wg(d.L), wu(d.L), wd(d.L);
  for (std::size_t l = 0; l < d.L; ++l) {
    const Layer& w = layers[l];
    wq[l] = {QType::Q4_0, w.q.data(), d.D, d.D};
    wk[l] = {w.kt, w.k.data(), kvd, d.D};
    wv[l] = {QType::Q4_0, w.v.data(), kvd, d.D};
    wo[l] = {QType::Q4_0, w.o.data(), d.D, d.D};
    wg[l] = {QType::Q4_0, w.gate.data(), d.F, d.D};
    wu[l] = {QType::Q4_0, w.up.data(), d.F, d.D};
    wd[l] = {QType::Q4_0, w.down.data(), d.D, d.F};
  }
  const WeightView emb{QType::BF16, embed.data(), d.V, d.D}, head{QType::Q8_0, lm.data(), d.V, d.D};
  std::vector<float> inv(d.hd / 2), cs(64 * d.hd / 2), sn(64 * d.hd / 2);
  efo_rope_table(inv.data(), cs.data(), sn.data(), 64, d.hd, 10000.0f);
  std::vector<float> kc(d.L * ids.size() * kvd, 0.f), vc(kc.size(), 0.f);
  std::vector<float> x(d.D), h(d.D), q(d.D), ctx(d.D), o(d.D), gate(d.F), up(d.F), logits(d.V), scores(ids.size());
  double worst = 0.0;
  bool argmax_same = true;
  for (std::size_t pos = 0; pos < ids.size(); ++pos) {
    ef::hip::row_f32(x.data(), emb, static_cast<std::size_t>(ids[pos]));
    for (std::size_t l = 0; l < d.L; ++l) {
      float* kl = kc.data() + l * ids.size() * kvd;
      float* vl = vc.data() + l * ids.size() * kvd;
      efo_rmsnorm(h.data(), x.data(), layers[l].an.data(), d.D, 1e-5f);
      const ef::kern::MatvecJob qkv[3] = {{q.data(), &wq[l], h.data()}, {kl + pos * kvd, &wk[l], h.data()},
                                          {vl + pos * kvd, &wv[l], h.data()}};
      ef::hip::matvec_jobs(qkv, 3, nullptr);
      efo_rope_apply(q.data(), d.H, d.hd, cs.data() + pos * d.hd / 2, sn.data() + pos * d.hd / 2);
      efo_rope_apply(kl + pos * kvd, d.KV, d.hd, cs.data() + pos * d.hd / 2, sn.data() + pos * d.hd / 2);
      efo_attention_heads(ctx.data(), q.data(), kl, vl, pos + 1, d.H, d.KV, d.hd, scores.data(), 0, d.H);
      ef::hip::matvec(o.data(), wo[l], ctx.data());
      efo_add_inplace(x.data(), o.data(), d.D);
      efo_rmsnorm(h.data(), x.data(), layers[l].fn.data(), d.D, 1e-5f);
      const ef::kern::MatvecJob gu[2] = {{gate.data(), &wg[l], h.data()}, {up.data(), &wu[l], h.data()}};
      ef::hip::matvec_jobs(gu, 2, nullptr);
      efo_swiglu(gate.data(), gate.data(), up.data(), d.F);
      ef::hip::matvec(o.data(), wd[l], gate.data());
      efo_add_inplace(x.data(), o.data(), d.D);
    }
    efo_rmsnorm(h.data(), x.data(), fnorm.data(), d.D, 1e-5f);
    ef::hip::matvec(logits.data(), head, h.data());
    ef::hip::throw_if_error();
    int err = 0;
    const float* ref = efo_transformer_forward(ot, ids[pos], pos, 1, &err);
    double mx = 0.0, mref = 1.0;
    for (std::size_t i = 0; i < d.V; ++i) {
      mx = std::max(mx, std::fabs(static_cast<double>(logits[i]) - ref[i]));
      mref = std::max(mref, std::fabs(static_cast<double>(ref[i])));
    }
    worst = std::max(worst, mx / mref);
    argmax_same = argmax_same && ef::hip::argmax(logits.data(), d.V) == efo_argmax(ref, d.V);
  }
  std::printf("shim forward vs oracle Transformer: max rel logit error %.3e\n", worst);
  check(worst < 1e-4, "logits within 1e-4 of the oracle at every position");
  check(argmax_same, "ef::hip::argmax equals kern::argmax at every position");

  // sampler: same ids as the oracle's restatement of ef::Sampler, draws advancing in step
  const ef::SamplerConfig sc{0.8f, 40, 0.95f, 1.1f, 7};
  ef::hip::Sampler gs(sc);
  const efo_sampler_config oc{0.8f, 40, 0.95f, 1.1f, 7};
  efo_sampler* os = efo_sampler_create(&oc);
  std::vector<std::int32_t> hist(ids.begin(), ids.end());
  bool same = true;
  std::vector<float> lg(32000);
  for (int step = 0; step < 20; ++step) {
    for (auto& v : lg) v = 3.0f * nd(g);
    const std::int32_t a = gs.sample(lg.data(), lg.size(), hist);
    const std::int32_t b = efo_sampler_sample(os, lg.data(), lg.size(), hist.data(), hist.size());
    same = same && a == b;
    hist.push_back(a);
  }
  check(same, "ef::hip::Sampler ids equal ef::Sampler's over 20 steps");
  bool threw = false;
  try {
    gs.sample(lg.data(), 0, hist);
  } catch (const ef::Error&) {
    threw = true;
  }
  check(threw, "empty vocabulary throws ef::Error (src/sampler.cpp:14)");

  // every storage type goes through the GPU GEMV: the BF16 embedding as a matrix (tied lm_head)
  std::vector<float> ye(d.V);
  ef::hip::matvec(ye.data(), emb, x.data());
  ef::hip::throw_if_error();
  double bf_err = 0.0;
  for (std::size_t r = 0; r < d.V; ++r) {
    const float want = efo_dot_bf16_avx2(reinterpret_cast<const std::uint16_t*>(embed.data()) + r * d.D, x.data(), d.D);
    bf_err = std::max(bf_err, std::fabs(static_cast<double>(ye[r]) - want));
  }
  check(bf_err <= 1e-4, "BF16 matvec within 1e-4 of dot_bf16_avx2");

  // noexcept GEMV failures are sticky and surface as ef::Error: a Q4_0 row longer than the GPU
  // kernels take (14336 columns)
  const std::size_t wide = 14368;
  std::vector<std::uint8_t> wb(wide / 32 * 18, 0x88);
  std::vector<float> xw(wide, 1.0f);
  float y1 = 0.0f;
  ef::hip::matvec(&y1, WeightView{QType::Q4_0, wb.data(), 1, wide}, xw.data());
  threw = false;
  try {
    ef::hip::throw_if_error();
  } catch (const ef::Error& e) {
    threw = std::string(e.what()).find("cols must be") != std::string::npos;
  }
  check(threw, "rejected launch -> sticky error -> ef::Error");
  efo_sampler_destroy(os);
  efo_transformer_destroy(ot);
  std::printf(fails ? "FAILED (%d)\n" : "OK\n", fails);
  return fails ? 1 : 0;
}
