// iek_bench_compare — the reference's bench_compare CLI (src/bin/bench_compare.rs) over the C ABI:
// cold start, interactive TTFT and decode throughput, each repeated --runs (>= 5) times, with the
// reference's median / p95 / min / max summaries and the --min-decode-tps gate.
//
//   iek_bench_compare [--model PATH] [--prompt-ids 1,2,3 | --prompt-tokens N [--seed S]] [--json]
//                     [--runs N] [--min-decode-tps X] [--device D]
//                     all [--decode-tokens N] | cold-start | interactive-ttft |
//                     decode-throughput [-n N]
//
// There is no tokenizer on this path: the prompt is given as token ids (or N seeded uniform ids in
// [1, vocab)), and the tokenizer regions of the reference (tokenizer_load_ms, tokenizer_encode_ms)
// are reported as 0. Regions (src/bench_metrics.rs:36-80):
//   cold:        gguf_metadata_ms, config_and_resolve_ms, tensor_load_ms (file -> HBM),
//                weights_build_ms, kv_alloc_ms (session create), prefill_prepare_ms (embedding
//                rows), prompt_eval_ms (prefill_forward), lm_head_sample_ms (final norm + LM head
//                + greedy argmax), cold_ttft_ms (wall from load start to the first token id)
//   interactive: weights resident, fresh KV (session reset): prefill_prepare_ms + prompt_eval_ms
//                + lm_head_sample_ms = ttft_infer_ms
//   decode:      warm prefill, then decode_tokens greedy steps (the captured-graph loop)
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "iek.h"

namespace {

using Clock = std::chrono::steady_clock;

double ms_since(Clock::time_point t0) { return std::chrono::duration<double, std::milli>(Clock::now() - t0).count(); }

[[noreturn]] void die(const std::string& m, int code = 1) {
  fprintf(stderr, "error: %s\n", m.c_str());
  exit(code);
}

void ok(iek_status st, const char* what) {
  if (st != IEK_OK) die(std::string(what) + ": " + iek_last_error(), (int)st);
}

struct Cold {
  size_t prompt_token_count = 0;
  double gguf_metadata_ms = 0, tokenizer_load_ms = 0, tokenizer_encode_ms = 0, config_and_resolve_ms = 0,
         tensor_load_ms = 0, prefill_prepare_ms = 0, weights_build_ms = 0, kv_alloc_ms = 0, prompt_eval_ms = 0,
         lm_head_sample_ms = 0, cold_ttft_ms = 0;
};
struct Inter {
  size_t prompt_token_count = 0;
  double tokenizer_encode_ms = 0, prefill_prepare_ms = 0, prompt_eval_ms = 0, lm_head_sample_ms = 0,
         ttft_infer_ms = 0, ttft_with_tokenizer_ms = 0;
};
struct Decode {
  size_t prompt_token_count = 0, decode_tokens = 0;
  double warm_prefill_ms = 0, decode_elapsed_ms = 0, decode_tokens_per_sec = 0;
};

struct Args {
  std::string model = "model/mistral-7b-v0.1/mistral-7b-v0.1.Q4_K_M.gguf";
  std::vector<uint32_t> prompt_ids;
  size_t prompt_tokens = 0;
  unsigned seed = 0;
  bool json = false;
  size_t runs = 5;
  bool have_min = false;
  double min_decode_tps = 0;
  int device = 0;
  std::string suite;
  size_t decode_tokens = 128;
};

// prompt_eval + first token on a session holding a fresh cache: embed, prefill_forward, greedy
void timed_prefill(iek_session* s, const std::vector<uint32_t>& ids, double* prep, double* eval, double* head) {
  auto t0 = Clock::now();
  ok(iek_session_embed(s, ids.data(), ids.size()), "embed");
  *prep = ms_since(t0);
  t0 = Clock::now();
  ok(iek_session_prefill_forward(s), "prefill_forward");
  *eval = ms_since(t0);
  t0 = Clock::now();
  uint32_t tok = 0;
  ok(iek_greedy_next_token(s, &tok), "greedy_next_token");
  *head = ms_since(t0);
}

// run_cold_start (bench_metrics.rs:199-296): from the start of the load to the first token id
Cold run_cold(const Args& a, const std::vector<uint32_t>& ids) {
  Cold c;
  c.prompt_token_count = ids.size();
  auto wall = Clock::now();
  iek_model* m = nullptr;
  ok(iek_model_load(a.model.c_str(), a.device, &m), "model load");
  iek_load_timings lt;
  ok(iek_model_load_timings(m, &lt), "load timings");
  c.gguf_metadata_ms = lt.gguf_metadata_ms;
  c.config_and_resolve_ms = lt.config_and_resolve_ms;
  c.tensor_load_ms = lt.tensor_load_ms;
  c.weights_build_ms = lt.weights_build_ms;
  auto t0 = Clock::now();
  iek_session* s = nullptr;
  ok(iek_session_create(m, &s), "session create");
  c.kv_alloc_ms = ms_since(t0);
  timed_prefill(s, ids, &c.prefill_prepare_ms, &c.prompt_eval_ms, &c.lm_head_sample_ms);
  c.cold_ttft_ms = ms_since(wall);
  iek_session_free(s);
  iek_model_free(m);
  return c;
}

// EngineBench::run_interactive_ttft (bench_metrics.rs:114-152) on a warm session: a fresh KV cache
// is a reset one (positions restart at 0; stale rows are never read)
Inter run_inter(iek_session* s, const std::vector<uint32_t>& ids) {
  Inter r;
  r.prompt_token_count = ids.size();
  ok(iek_session_reset(s), "reset");
  timed_prefill(s, ids, &r.prefill_prepare_ms, &r.prompt_eval_ms, &r.lm_head_sample_ms);
  r.ttft_infer_ms = r.prefill_prepare_ms + r.prompt_eval_ms + r.lm_head_sample_ms;
  r.ttft_with_tokenizer_ms = r.ttft_infer_ms + r.tokenizer_encode_ms;
  return r;
}

// EngineBench::run_decode_throughput (bench_metrics.rs:156-196): warm prefill untimed, then n
// greedy steps (logits -> argmax -> embedding -> decode_forward), replayed as one graph
Decode run_decode(iek_session* s, const std::vector<uint32_t>& ids, size_t n) {
  if (n == 0) die("decode_throughput: decode_tokens must be > 0", IEK_ERR_MODEL);
  Decode d;
  d.prompt_token_count = ids.size();
  d.decode_tokens = n;
  auto t0 = Clock::now();
  ok(iek_session_reset(s), "reset");
  ok(iek_session_prefill(s, ids.data(), ids.size()), "prefill");
  d.warm_prefill_ms = ms_since(t0);
  std::vector<uint32_t> out(n);
  t0 = Clock::now();
  ok(iek_session_generate_greedy(s, n, out.data()), "generate_greedy");
  d.decode_elapsed_ms = ms_since(t0);
  d.decode_tokens_per_sec = (double)n / std::max(d.decode_elapsed_ms / 1e3, 1e-300);
  return d;
}

void finite_pos(double x, const char* name) {
  if (!std::isfinite(x)) die(std::string(name) + " is not finite", IEK_ERR_MODEL);
  if (x < 0) die(std::string(name) + " is negative", IEK_ERR_MODEL);
}
void check_cold(const Cold& c) {
  finite_pos(c.gguf_metadata_ms, "cold.gguf_metadata_ms");
  finite_pos(c.cold_ttft_ms, "cold.cold_ttft_ms");
  finite_pos(c.lm_head_sample_ms, "cold.lm_head_sample_ms");
  if (c.prompt_token_count == 0) die("cold.prompt_token_count is zero", IEK_ERR_MODEL);
}
void check_inter(const Inter& m) {
  finite_pos(m.ttft_infer_ms, "interactive.ttft_infer_ms");
  finite_pos(m.ttft_with_tokenizer_ms, "interactive.ttft_with_tokenizer_ms");
  if (m.prompt_token_count == 0) die("interactive.prompt_token_count is zero", IEK_ERR_MODEL);
}
void check_decode(const Decode& d, const Args& a) {
  finite_pos(d.decode_elapsed_ms, "decode.decode_elapsed_ms");
  if (!std::isfinite(d.decode_tokens_per_sec)) die("decode.decode_tokens_per_sec is not finite", IEK_ERR_MODEL);
  if (d.decode_tokens == 0) die("decode.decode_tokens is zero", IEK_ERR_MODEL);
  if (a.have_min && d.decode_tokens_per_sec < a.min_decode_tps) {
    char b[160];
    snprintf(b, sizeof b, "decode.decode_tokens_per_sec %.3f < --min-decode-tps %.3f", d.decode_tokens_per_sec,
             a.min_decode_tps);
    die(b, IEK_ERR_MODEL);
  }
}

// median / percentile as bench_compare.rs:220-242 (even count: mean of the middle two; percentile
// rank = round((n - 1) p) of the sorted values)
double median(std::vector<double> v) {
  if (v.empty()) return 0;
  std::sort(v.begin(), v.end());
  size_t n = v.size();
  return n % 2 ? v[n / 2] : (v[n / 2 - 1] + v[n / 2]) / 2.0;
}
double percentile(std::vector<double> v, double p) {
  if (v.empty()) return 0;
  std::sort(v.begin(), v.end());
  return v[(size_t)std::llround((double)(v.size() - 1) * p)];
}

std::string num(double x) {
  char b[64];
  snprintf(b, sizeof b, "%.6f", x);
  return b;
}
std::string stats(const std::vector<double>& v, bool p95) {
  std::string s = "{\"median\": " + num(median(v));
  if (p95) s += ", \"p95\": " + num(percentile(v, 0.95));
  s += ", \"min\": " + num(*std::min_element(v.begin(), v.end()));
  s += ", \"max\": " + num(*std::max_element(v.begin(), v.end())) + "}";
  return s;
}

std::string json_cold(const Cold& c) {
  return "{\"prompt_token_count\": " + std::to_string(c.prompt_token_count) +
         ", \"gguf_metadata_ms\": " + num(c.gguf_metadata_ms) + ", \"tokenizer_load_ms\": " + num(c.tokenizer_load_ms) +
         ", \"tokenizer_encode_ms\": " + num(c.tokenizer_encode_ms) +
         ", \"config_and_resolve_ms\": " + num(c.config_and_resolve_ms) + ", \"tensor_load_ms\": " +
         num(c.tensor_load_ms) + ", \"prefill_prepare_ms\": " + num(c.prefill_prepare_ms) +
         ", \"weights_build_ms\": " + num(c.weights_build_ms) + ", \"kv_alloc_ms\": " + num(c.kv_alloc_ms) +
         ", \"prompt_eval_ms\": " + num(c.prompt_eval_ms) + ", \"lm_head_sample_ms\": " + num(c.lm_head_sample_ms) +
         ", \"cold_ttft_ms\": " + num(c.cold_ttft_ms) + "}";
}
std::string json_inter(const Inter& m) {
  return "{\"prompt_token_count\": " + std::to_string(m.prompt_token_count) +
         ", \"tokenizer_encode_ms\": " + num(m.tokenizer_encode_ms) + ", \"prefill_prepare_ms\": " +
         num(m.prefill_prepare_ms) + ", \"prompt_eval_ms\": " + num(m.prompt_eval_ms) +
         ", \"lm_head_sample_ms\": " + num(m.lm_head_sample_ms) + ", \"ttft_infer_ms\": " + num(m.ttft_infer_ms) +
         ", \"ttft_with_tokenizer_ms\": " + num(m.ttft_with_tokenizer_ms) + "}";
}
std::string json_decode(const Decode& d) {
  return "{\"prompt_token_count\": " + std::to_string(d.prompt_token_count) +
         ", \"decode_tokens\": " + std::to_string(d.decode_tokens) + ", \"warm_prefill_ms\": " +
         num(d.warm_prefill_ms) + ", \"decode_elapsed_ms\": " + num(d.decode_elapsed_ms) +
         ", \"decode_tokens_per_sec\": " + num(d.decode_tokens_per_sec) + "}";
}
template <class T, class F>
std::string json_list(const std::vector<T>& v, F f) {
  std::string s = "[";
  for (size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + f(v[i]);
  return s + "]";
}
std::string summary_inter(const std::vector<Inter>& r) {
  std::vector<double> t, p;
  for (auto& m : r) {
    t.push_back(m.ttft_infer_ms);
    p.push_back(m.prompt_eval_ms);
  }
  return "{\"runs\": " + std::to_string(r.size()) + ", \"ttft_infer_ms\": " + stats(t, false) +
         ", \"prompt_eval_ms\": " + stats(p, false) + "}";
}
std::string summary_decode(const std::vector<Decode>& r) {
  std::vector<double> t, e;
  for (auto& d : r) {
    t.push_back(d.decode_tokens_per_sec);
    e.push_back(d.decode_elapsed_ms);
  }
  return "{\"runs\": " + std::to_string(r.size()) + ", \"decode_tokens_per_sec\": " + stats(t, true) +
         ", \"decode_elapsed_ms\": " + stats(e, false) + "}";
}

void print_cold(const Cold& c) {
  printf("=== cold-start ===\n");
  printf("  prompt_token_count: %zu\n", c.prompt_token_count);
  printf("  gguf_metadata_ms:   %.3f\n", c.gguf_metadata_ms);
  printf("  config_resolve_ms:  %.3f\n", c.config_and_resolve_ms);
  printf("  tensor_load_ms:     %.3f  (mapped file -> HBM)\n", c.tensor_load_ms);
  printf("  weights_build_ms:   %.3f\n", c.weights_build_ms);
  printf("  kv_alloc_ms:        %.3f\n", c.kv_alloc_ms);
  printf("  prefill_prepare_ms: %.3f\n", c.prefill_prepare_ms);
  printf("  prompt_eval_ms:     %.3f\n", c.prompt_eval_ms);
  printf("  lm_head_sample_ms:  %.3f\n", c.lm_head_sample_ms);
  printf("  cold_ttft_ms:       %.3f\n", c.cold_ttft_ms);
}
void print_inter(const Inter& m) {
  printf("=== interactive-ttft (warm weights, fresh KV) ===\n");
  printf("  prompt_token_count:        %zu\n", m.prompt_token_count);
  printf("  prefill_prepare_ms:        %.3f\n", m.prefill_prepare_ms);
  printf("  prompt_eval_ms:            %.3f\n", m.prompt_eval_ms);
  printf("  lm_head_sample_ms:         %.3f\n", m.lm_head_sample_ms);
  printf("  ttft_infer_ms:             %.3f\n", m.ttft_infer_ms);
}
void print_decode(const Decode& d) {
  printf("=== decode-throughput ===\n");
  printf("  prompt_token_count:   %zu\n", d.prompt_token_count);
  printf("  decode_tokens:        %zu\n", d.decode_tokens);
  printf("  warm_prefill_ms:      %.3f\n", d.warm_prefill_ms);
  printf("  decode_elapsed_ms:    %.3f\n", d.decode_elapsed_ms);
  printf("  decode_tokens_per_sec:%.3f\n", d.decode_tokens_per_sec);
  printf("  prefill_tokens_per_s: %.3f  (rough pp analog)\n",
         (double)d.prompt_token_count / std::max(d.warm_prefill_ms / 1e3, 2.220446049250313e-16));
}

Args parse(int argc, char** argv) {
  Args a;
  auto need = [&](int& i) -> const char* {
    if (i + 1 >= argc) die(std::string("missing value for ") + argv[i], 2);
    return argv[++i];
  };
  for (int i = 1; i < argc; ++i) {
    std::string o = argv[i];
    if (o == "-m" || o == "--model") a.model = need(i);
    else if (o == "--prompt-ids") {
      std::string s = need(i);
      size_t p = 0;
      while (p < s.size()) {
        size_t q = s.find(',', p);
        if (q == std::string::npos) q = s.size();
        if (q > p) a.prompt_ids.push_back((uint32_t)strtoul(s.substr(p, q - p).c_str(), nullptr, 10));
        p = q + 1;
      }
    } else if (o == "--prompt-tokens") a.prompt_tokens = strtoull(need(i), nullptr, 10);
    else if (o == "--seed") a.seed = (unsigned)strtoul(need(i), nullptr, 10);
    else if (o == "--json") a.json = true;
    else if (o == "--runs") a.runs = strtoull(need(i), nullptr, 10);
    else if (o == "--min-decode-tps") {
      a.have_min = true;
      a.min_decode_tps = strtod(need(i), nullptr);
    } else if (o == "--device") a.device = atoi(need(i));
    else if (o == "--decode-tokens" || o == "-n") a.decode_tokens = strtoull(need(i), nullptr, 10);
    else if (o == "all" || o == "cold-start" || o == "interactive-ttft" || o == "decode-throughput") a.suite = o;
    else if (o == "-h" || o == "--help") {
      printf("usage: %s [--model PATH] [--prompt-ids 1,2,3 | --prompt-tokens N [--seed S]] [--json] [--runs N]\n"
             "          [--min-decode-tps X] [--device D] all [--decode-tokens N] | cold-start |\n"
             "          interactive-ttft | decode-throughput [-n N]\n",
             argv[0]);
      exit(0);
    } else die("unknown argument " + o, 2);
  }
  if (a.suite.empty()) die("a subcommand is required: all, cold-start, interactive-ttft or decode-throughput", 2);
  if (a.runs < 5) die("--runs must be at least 5 for stable comparisons", IEK_ERR_MODEL);
  return a;
}

}  // namespace

int main(int argc, char** argv) {
  Args a = parse(argc, argv);
  // the prompt: explicit ids, or seeded uniform ids in [1, vocab) once the vocabulary is known
  iek_model* model = nullptr;
  ok(iek_model_load(a.model.c_str(), a.device, &model), "model load");
  iek_model_config cfg;
  ok(iek_model_config_get(model, &cfg), "config");
  std::vector<uint32_t> ids = a.prompt_ids;
  if (ids.empty()) {
    const size_t n = a.prompt_tokens ? a.prompt_tokens : 512;
    std::mt19937 rng(a.seed);
    std::uniform_int_distribution<uint32_t> pick(1, (uint32_t)cfg.vocab_size - 1);
    for (size_t i = 0; i < n; ++i) ids.push_back(pick(rng));
  }
  iek_session* sess = nullptr;
  ok(iek_session_create(model, &sess), "session create");
  // one untimed pass so that kernels and the decode graph are resident before the timed runs
  if (a.suite != "cold-start") {
    Inter w = run_inter(sess, ids);
    (void)w;
    if (a.suite != "interactive-ttft") (void)run_decode(sess, ids, std::min<size_t>(a.decode_tokens, 8));
  }
  std::vector<Cold> cold;
  std::vector<Inter> inter;
  std::vector<Decode> dec;
  for (size_t r = 0; r < a.runs; ++r) {
    if (a.suite == "all" || a.suite == "cold-start") {
      cold.push_back(run_cold(a, ids));
      check_cold(cold.back());
    }
    if (a.suite == "all" || a.suite == "interactive-ttft") {
      inter.push_back(run_inter(sess, ids));
      check_inter(inter.back());
    }
    if (a.suite == "all" || a.suite == "decode-throughput") {
      dec.push_back(run_decode(sess, ids, a.decode_tokens));
      check_decode(dec.back(), a);
    }
  }
  iek_session_free(sess);
  iek_model_free(model);
  std::string prompt = json_list(ids, [](uint32_t x) { return std::to_string(x); });
  if (a.json) {
    std::string head = "{\"suite\": \"" + a.suite + "\", \"model\": \"" + a.model + "\", \"tokenizer\": null, " +
                       "\"prompt_ids\": " + prompt;
    if (a.suite == "all") {
      printf("%s, \"runs\": {\"cold\": %s, \"interactive\": %s, \"decode\": %s}, \"summary\": {\"interactive\": %s, "
             "\"decode\": %s}}\n",
             head.c_str(), json_list(cold, json_cold).c_str(), json_list(inter, json_inter).c_str(),
             json_list(dec, json_decode).c_str(), summary_inter(inter).c_str(), summary_decode(dec).c_str());
    } else if (a.suite == "cold-start") {
      printf("%s, \"runs\": %s}\n", head.c_str(), json_list(cold, json_cold).c_str());
    } else if (a.suite == "interactive-ttft") {
      printf("%s, \"runs\": %s, \"summary\": %s}\n", head.c_str(), json_list(inter, json_inter).c_str(),
             summary_inter(inter).c_str());
    } else {
      printf("%s, \"runs\": %s, \"summary\": %s}\n", head.c_str(), json_list(dec, json_decode).c_str(),
             summary_decode(dec).c_str());
    }
  } else {
    if (!cold.empty()) print_cold(cold[0]);
    if (!inter.empty()) print_inter(inter[0]);
    if (!dec.empty()) print_decode(dec[0]);
    printf("=== summary over %zu runs ===\n", a.runs);
    if (!inter.empty()) printf("  interactive: %s\n", summary_inter(inter).c_str());
    if (!dec.empty()) printf("  decode:      %s\n", summary_decode(dec).c_str());
    if (a.have_min && a.suite != "all" && a.suite != "decode-throughput")
      fprintf(stderr, "warning: --min-decode-tps ignored for %s\n", a.suite.c_str());
  }
  return 0;
}
