// The C++ mirror of the crate's API (include/orda/orda.hpp) exercised the way
// the crate's own tests use the Rust API (tests/end_to_end.rs).
//
//   api_test cpu          checks that need no GPU; prints a JSON object of
//                         values for the caller to compare with the oracle
//   api_test gpu OUTDIR   the reference's end-to-end scenarios on the GPU: the
//                         assertions tests/end_to_end.rs makes without an f64
//                         forward (chunk invariance, component identity,
//                         sum = mean * n, INT8 close but lossy, pure student
//                         CE), and the outputs of its gradient scenarios
//                         written to OUTDIR for comparison with the oracle
//
// Exit status 0 when every check passed; failed checks are listed under
// "failures" in the JSON printed on stdout.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "orda/orda.hpp"

namespace {

std::vector<std::string> g_failures;

void expect(bool ok, const std::string& what) {
  if (!ok) g_failures.push_back(what);
}

// tests/end_to_end.rs:14-27 (a 64-bit LCG; the f32 arithmetic as written there)
std::vector<float> fill(size_t n, uint64_t seed, float scale) {
  uint64_t s = seed * 2862933555777941757ull + 3037000493ull;
  std::vector<float> out(n);
  for (size_t i = 0; i < n; ++i) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    const float u = static_cast<float>(s >> 33) / static_cast<float>(1ull << 31);
    out[i] = (u * 2.0f - 1.0f) * scale;
  }
  return out;
}

// tests/end_to_end.rs:29-36
std::vector<int64_t> labels(size_t bt, size_t v, size_t ignore_every, int64_t ignore_index) {
  std::vector<int64_t> out(bt);
  for (size_t i = 0; i < bt; ++i)
    out[i] = ignore_every && i % ignore_every == 0 ? ignore_index
                                                    : static_cast<int64_t>((i * 7 + 3) % v);
  return out;
}

orda::Mat mat(size_t rows, size_t cols, uint64_t seed, float scale) {
  return orda::Mat::from_vec(rows, cols, fill(rows * cols, seed, scale));
}

// tests/end_to_end.rs:80-87
orda::LossOptions base_opts() {
  orda::LossOptions o;
  o.student_ce_weight = 1.0f;
  o.kd_weight = 0.5f;
  o.temperature = 1.5f;
  return o;
}

std::string num(double x) {
  char b[64];
  snprintf(b, sizeof b, "%.9g", x);
  return b;
}

std::string json_list(const std::vector<size_t>& v) {
  std::string s = "[";
  for (size_t i = 0; i < v.size(); ++i) s += (i ? "," : "") + std::to_string(v[i]);
  return s + "]";
}

std::string quoted(const std::string& s) {
  std::string o = "\"";
  for (char c : s) o += c == '"' || c == '\\' ? std::string("\\") + c : std::string(1, c);
  return o + "\"";
}

int finish(std::string body) {
  std::string f = "[";
  for (size_t i = 0; i < g_failures.size(); ++i) f += (i ? "," : "") + quoted(g_failures[i]);
  f += "]";
  printf("{%s%s\"failures\": %s}\n", body.c_str(), body.empty() ? "" : ", ", f.c_str());
  return g_failures.empty() ? 0 : 1;
}

template <class F>
std::string error_of(F&& f, int32_t* status = nullptr) {
  try {
    f();
  } catch (const orda::Error& e) {
    if (status) *status = e.status();
    return e.what();
  }
  return "";
}

int run_cpu() {
  std::string body;
  // LossOptions::default (src/api.rs:49-64), KernelConfig presets
  const orda::LossOptions d;
  expect(d.student_ce_weight == 1.0f && !d.teacher_ce_weight && d.kd_weight == 0.0f &&
             d.temperature == 1.0f && d.ignore_index == -100 && d.label_smoothing == 0.0f &&
             d.reduction == orda::Reduction::Mean && d.chunk_size == orda::ChunkSize::Auto() &&
             d.backend == orda::Backend::Auto,
         "LossOptions defaults");
  orda_loss_options c{};
  orda_loss_options_default(&c);
  const orda_loss_options m = d.to_c();
  expect(c.student_ce_weight == m.student_ce_weight && c.has_teacher_ce_weight == m.has_teacher_ce_weight &&
             c.kd_weight == m.kd_weight && c.temperature == m.temperature &&
             c.ignore_index == m.ignore_index && c.reduction == m.reduction &&
             c.chunk_fixed == m.chunk_fixed && c.backend == m.backend &&
             c.config.max_fused_size == m.config.max_fused_size && c.config.profile == m.config.profile,
         "LossOptions defaults equal the C ABI's");
  const auto fast = orda::KernelConfig::from_profile(orda::Profile::Fast);
  const auto bal = orda::KernelConfig::from_profile(orda::Profile::Balanced);
  const auto dbg = orda::KernelConfig::from_profile(orda::Profile::Debug);
  expect(fast.fast_math && fast.fast_math_exp() && fast.fast_math_log() && fast.fast_math_mul(),
         "Profile::Fast sets fast_math");
  expect(!bal.fast_math && !dbg.fast_math && dbg.profile == orda::Profile::Debug,
         "Balanced and Debug leave fast_math off");
  expect(bal.max_fused_size == orda::DEFAULT_MAX_FUSED_SIZE && !bal.max_chunks &&
             !bal.stochastic_seed && !bal.quantize_grad_weight,
         "KernelConfig::default fields");
  // KernelConfig::validate (src/config.rs:106-119)
  orda::KernelConfig k;
  k.max_fused_size = 3;
  body += "\"validate_max_fused_size\": " + quoted(error_of([&] { k.validate(); }));
  k.max_fused_size = 1024;
  k.max_chunks = 0;
  body += ", \"validate_max_chunks\": " + quoted(error_of([&] { k.validate(); }));
  k.max_chunks = 4;
  expect(error_of([&] { k.validate(); }).empty(), "a valid config validates");
  expect(orda::is_power_of_two(1) && orda::is_power_of_two(4096) && !orda::is_power_of_two(0) &&
             !orda::is_power_of_two(6),
         "is_power_of_two");
  // the resolver (src/resolver.rs), values for the oracle to check
  body += ", \"plans\": [";
  const size_t bts[] = {1, 7, 256, 2048, 4096, 8192, 100000};
  bool first = true;
  for (size_t bt : bts)
    for (int fixed = 0; fixed < 2; ++fixed)
      for (int hv = 0; hv < 2; ++hv)
        for (int hm = 0; hm < 2; ++hm) {
          const auto cs = fixed ? orda::ChunkSize::Fixed(bt / 3 + 1) : orda::ChunkSize::Auto();
          const std::optional<size_t> v = hv ? std::optional<size_t>(131072) : std::nullopt;
          const std::optional<size_t> mc = hm ? std::optional<size_t>(8) : std::nullopt;
          const auto p = orda::resolve_chunk_size(bt, cs, v, mc);
          body += std::string(first ? "" : ",") + "[" + std::to_string(bt) + "," +
                  std::to_string(fixed) + "," + std::to_string(hv) + "," + std::to_string(hm) +
                  "," + std::to_string(p.chunk_size) + "," + std::to_string(p.num_chunks) + "]";
          first = false;
        }
  body += "]";
  body += ", \"schedule_8192\": " +
          json_list(orda::chunk_doubling_schedule(8192, 16, orda::default_max_chunks_limit(8192)));
  body += ", \"schedule_1000_3\": " + json_list(orda::chunk_doubling_schedule(1000, 3, 1000));
  body += ", \"default_max_chunks_limit\": " + json_list({orda::default_max_chunks_limit(1),
                                                         orda::default_max_chunks_limit(8192),
                                                         orda::default_max_chunks_limit(100000)});
  body += ", \"chunks_from_raw\": " + json_list({orda::chunks_from_raw(0.5), orda::chunks_from_raw(1.5),
                                                 orda::chunks_from_raw(3.0), orda::chunks_from_raw(100.0)});
  body += ", \"ceil_div\": " + json_list({orda::ceil_div(10, 3), orda::ceil_div(9, 3)});
  int32_t st = 0;
  body += ", \"resolve_bt0\": " +
          quoted(error_of([&] { orda::resolve_chunk_size(0, orda::ChunkSize::Auto(), {}, {}); }, &st));
  expect(st == ORDA_ERR_INVALID, "resolve_chunk_size(0) is an invalid-argument error");
  // Mat (src/mat.rs)
  bool threw = false;
  try {
    orda::Mat::from_vec(2, 3, std::vector<float>(5));
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  expect(threw, "Mat::from_vec rejects a wrong length");
  const auto z = orda::Mat::zeros(2, 3);
  expect(z.shape() == std::make_pair(size_t{2}, size_t{3}) && z.get(1, 2) == 0.0f, "Mat::zeros");
  // Teacher (src/teacher.rs)
  const auto tt = orda::Teacher::Tied(orda::Mat::zeros(2, 3));
  const auto ts = orda::Teacher::Separate(orda::Mat::zeros(2, 3), orda::Mat::zeros(4, 3));
  const auto tp = orda::Teacher::Precomputed(orda::Mat::zeros(2, 4));
  expect(tt.mode() == orda::TeacherMode::Tied && tt.default_teacher_ce_weight() == 1.0f &&
             ts.default_teacher_ce_weight() == 0.0f && tp.default_teacher_ce_weight() == 0.0f,
         "Teacher modes and default teacher CE weights");
  // the GPU path (is_available() is false without a device: calls fail
  // with ORDA_ERR_UNAVAILABLE instead of falling back to the host)
  const bool avail = orda::is_available();
  body += std::string(", \"is_available\": ") + (avail ? "true" : "false");
  if (!avail) {
    st = 0;
    const std::string e = error_of(
        [&] {
          orda::distillation_loss(mat(4, 3, 1, 0.3f), mat(5, 3, 2, 0.2f), labels(4, 5, 0, -100),
                                  orda::Teacher::Tied(mat(4, 3, 3, 0.3f)), base_opts());
        },
        &st);
    expect(st == ORDA_ERR_UNAVAILABLE && !e.empty(), "without a GPU the loss fails as unavailable");
  }
  return finish(body);
}

bool write_mat(const std::string& path, const orda::Mat& m) {
  FILE* f = fopen(path.c_str(), "wb");
  if (!f) return false;
  const bool ok = fwrite(m.data.data(), sizeof(float), m.data.size(), f) == m.data.size();
  return fclose(f) == 0 && ok;
}

std::string dump(const std::string& dir, const std::string& name, const orda::DistillationLossOutput& o) {
  std::string s = quoted(name) + ": {\"loss\": " + num(o.loss) + ", \"student_ce\": " +
                  num(o.student_ce) + ", \"teacher_ce\": " + num(o.teacher_ce) + ", \"kl\": " +
                  num(o.kl) + ", \"chunk_plan\": " +
                  json_list({o.chunk_plan.chunk_size, o.chunk_plan.num_chunks});
  auto one = [&](const char* field, const orda::Mat& m) {
    const std::string file = name + "." + field + ".f32";
    expect(write_mat(dir + "/" + file, m), "write " + file);
    s += std::string(", \"") + field + "\": [" + quoted(file) + "," + std::to_string(m.rows) + "," +
         std::to_string(m.cols) + "]";
  };
  one("grad_student_hidden", o.grad_student_hidden);
  one("grad_weight", o.grad_weight);
  if (o.grad_teacher_hidden) one("grad_teacher_hidden", *o.grad_teacher_hidden);
  if (o.grad_teacher_weight) one("grad_teacher_weight", *o.grad_teacher_weight);
  return s + "}";
}

float max_abs_diff(const orda::Mat& a, const orda::Mat& b, float scale_b = 1.0f) {
  float m = 0.0f;
  for (size_t i = 0; i < a.data.size(); ++i) m = std::fmax(m, std::fabs(a.data[i] - b.data[i] * scale_b));
  return m;
}

int run_gpu(const std::string& dir) {
  using orda::LossOptions;
  using orda::Teacher;
  orda::Context ctx(0);
  std::string body = "\"scenarios\": {";
  // The gradient scenarios of tests/end_to_end.rs:89-204, written out for the
  // oracle comparison.
  {
    LossOptions o = base_opts();
    o.teacher_ce_weight = 1.0f;
    o.label_smoothing = 0.1f;
    body += dump(dir, "tied", orda::distillation_loss(&ctx, mat(6, 5, 1, 0.3f), mat(7, 5, 2, 0.2f),
                                                     labels(6, 7, 4, -100),
                                                     Teacher::Tied(mat(6, 5, 3, 0.3f)), o));
  }
  {
    LossOptions o = base_opts();
    o.teacher_ce_weight = 0.7f;
    body += ", " + dump(dir, "separate",
                        orda::distillation_loss(&ctx, mat(6, 5, 11, 0.3f), mat(7, 5, 12, 0.2f),
                                                labels(6, 7, 0, -100),
                                                Teacher::Separate(mat(6, 4, 13, 0.3f), mat(7, 4, 14, 0.2f)),
                                                o));
  }
  body += ", " + dump(dir, "precomputed",
                      orda::distillation_loss(&ctx, mat(6, 5, 21, 0.3f), mat(7, 5, 22, 0.2f),
                                              labels(6, 7, 5, -100),
                                              Teacher::Precomputed(mat(6, 7, 23, 0.5f)), base_opts()));
  // A shape that spans several GEMM tiles in every dimension.
  {
    LossOptions o = base_opts();
    o.teacher_ce_weight = 1.0f;
    o.label_smoothing = 0.1f;
    o.chunk_size = orda::ChunkSize::Fixed(100);
    body += ", " + dump(dir, "tied_300x70x1000",
                        orda::distillation_loss(&ctx, mat(300, 70, 81, 1.0f), mat(1000, 70, 82, 0.1f),
                                                labels(300, 1000, 9, -100),
                                                Teacher::Tied(mat(300, 70, 83, 1.0f)), o));
  }
  body += "}";

  // tests/end_to_end.rs:206-228: no teacher term
  {
    LossOptions o;
    o.kd_weight = 0.0f;
    o.teacher_ce_weight = 0.0f;
    const auto out = orda::distillation_loss(&ctx, mat(8, 4, 31, 0.3f), mat(6, 4, 32, 0.2f),
                                             labels(8, 6, 0, -100),
                                             Teacher::Tied(orda::Mat::zeros(8, 4)), o);
    expect(out.teacher_ce == 0.0f && out.kl == 0.0f, "pure student CE: no teacher term");
    expect(!out.grad_teacher_hidden && !out.grad_teacher_weight, "pure student CE: no teacher gradients");
  }
  // tests/end_to_end.rs:230-278: chunking is exact
  {
    const auto s = mat(16, 5, 41, 0.3f), w = mat(9, 5, 42, 0.2f);
    const auto t = Teacher::Tied(mat(16, 5, 43, 0.3f));
    const auto y = labels(16, 9, 3, -100);
    auto mk = [&](orda::ChunkSize cs) {
      LossOptions o = base_opts();
      o.chunk_size = cs;
      o.teacher_ce_weight = 1.0f;
      return orda::distillation_loss(&ctx, s, w, y, t, o);
    };
    const auto full = mk(orda::ChunkSize::Fixed(16));
    for (const auto& other : {mk(orda::ChunkSize::Fixed(1)), mk(orda::ChunkSize::Fixed(3)),
                              mk(orda::ChunkSize::Auto())}) {
      expect(std::fabs(full.loss - other.loss) < 1e-5f, "loss differs across chunking");
      expect(max_abs_diff(full.grad_weight, other.grad_weight) < 1e-5f, "grad_weight differs across chunking");
      expect(max_abs_diff(full.grad_student_hidden, other.grad_student_hidden) < 1e-5f,
             "grad_student_hidden differs across chunking");
    }
  }
  // tests/end_to_end.rs:280-311: total = w_s*student_ce + w_t*teacher_ce + kd*kl
  {
    LossOptions o;
    o.student_ce_weight = 1.0f;
    o.teacher_ce_weight = 0.8f;
    o.kd_weight = 0.5f;
    o.temperature = 2.0f;
    const auto out = orda::distillation_loss(&ctx, mat(10, 4, 51, 0.3f), mat(8, 4, 52, 0.2f),
                                             labels(10, 8, 0, -100),
                                             Teacher::Tied(mat(10, 4, 53, 0.3f)), o);
    const float recon = 1.0f * out.student_ce + 0.8f * out.teacher_ce + 0.5f * out.kl;
    expect(std::fabs(recon - out.loss) < 1e-4f, "loss components are inconsistent");
    body += ", \"components\": {\"loss\": " + num(out.loss) + "}";
  }
  // tests/end_to_end.rs:313-358: sum = mean * n_valid
  {
    const auto s = mat(8, 4, 61, 0.3f), w = mat(6, 4, 62, 0.2f);
    const auto t = Teacher::Tied(mat(8, 4, 63, 0.3f));
    const auto y = labels(8, 6, 4, -100);
    float n_valid = 0.0f;
    for (int64_t l : y) n_valid += l != -100;
    LossOptions om = base_opts(), os = base_opts();
    om.teacher_ce_weight = os.teacher_ce_weight = 1.0f;
    os.reduction = orda::Reduction::Sum;
    const auto mean = orda::distillation_loss(&ctx, s, w, y, t, om);
    const auto sum = orda::distillation_loss(&ctx, s, w, y, t, os);
    expect(std::fabs(sum.loss - mean.loss * n_valid) < 1e-3f, "sum loss is not mean * n");
    expect(max_abs_diff(sum.grad_weight, mean.grad_weight, n_valid) < 1e-3f,
           "sum gradients are not mean gradients * n");
  }
  // tests/end_to_end.rs:360-410: INT8 grad_W close but lossy, and the
  // quantizer entry point on the same gradient
  {
    const auto s = mat(8, 4, 71, 0.3f), w = mat(20, 4, 72, 0.2f);
    const auto t = Teacher::Tied(mat(8, 4, 73, 0.3f));
    const auto y = labels(8, 20, 0, -100);
    LossOptions oe = base_opts();
    oe.teacher_ce_weight = 1.0f;
    LossOptions oq = oe;
    oq.config.quantize_grad_weight = true;
    const auto exact = orda::distillation_loss(&ctx, s, w, y, t, oe);
    const auto quant = orda::distillation_loss(&ctx, s, w, y, t, oq);
    expect(std::fabs(exact.loss - quant.loss) < 1e-6f, "quantization changed the loss");
    const float d = max_abs_diff(exact.grad_weight, quant.grad_weight);
    expect(d > 0.0f && d < 0.05f, "INT8 grad_W is not close but lossy");
    const auto qd = orda::quant_dequant_grad_w(exact.grad_weight, y, -100, false, 0, 1.0f, &ctx);
    expect(qd.dequantized == quant.grad_weight,
           "the quantizer entry point differs from the loss's INT8 step");
    expect(write_mat(dir + "/quant.grad_w.f32", exact.grad_weight) &&
               write_mat(dir + "/quant.deq.f32", qd.dequantized),
           "write quant files");
    FILE* f = fopen((dir + "/quant.codes.i8").c_str(), "wb");
    expect(f && fwrite(qd.codes.data(), 1, qd.codes.size(), f) == qd.codes.size() && fclose(f) == 0,
           "write quant codes");
    orda::Mat sc = orda::Mat::from_vec(qd.scales.size(), 1, qd.scales);
    expect(write_mat(dir + "/quant.scales.f32", sc), "write quant scales");
  }
  // the chunk-launcher slot (src/cuda/launch.rs:51-158) on a row pair
  {
    const std::vector<float> lc = {0.1f, 0.2f, 0.3f, -1.0f, 2.0f, 1.0f, -0.5f, 0.0f, 0.7f, 0.2f};
    const auto r = orda::kl_ce_on_logits_chunk(lc, {4}, 1, 5, 5, 1.0f / 1.5f, 0.6f, 2.25f, 1.0f,
                                               1.0f, 0.1f, -100, false, true, &ctx);
    body += ", \"slot\": {\"kl_per_row\": " + num(r.kl_per_row[0]) + ", \"ce_loss\": [" +
            num(r.ce_loss[0]) + "," + num(r.ce_loss[1]) + "], \"grad_kl_student\": [";
    for (size_t i = 0; i < r.grad_kl_student.size(); ++i) body += (i ? "," : "") + num(r.grad_kl_student[i]);
    body += "], \"grad_ce\": [";
    for (size_t i = 0; i < r.grad_ce.size(); ++i) body += (i ? "," : "") + num(r.grad_ce[i]);
    body += "]}";
  }
  return finish(body);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc >= 2 && !strcmp(argv[1], "cpu")) return run_cpu();
  if (argc >= 3 && !strcmp(argv[1], "gpu")) {
    try {
      return run_gpu(argv[2]);
    } catch (const std::exception& e) {
      g_failures.push_back(std::string("exception: ") + e.what());
      return finish("");
    }
  }
  fprintf(stderr, "usage: %s cpu | gpu OUTDIR\n", argv[0]);
  return 2;
}
