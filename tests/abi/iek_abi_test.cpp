// C++ caller of the C ABI (include/iek.h), linked against the static libiek.a with g++: what a
// Rust crate's `static=iek` link sees. Drives load -> prefill -> greedy generation three ways
// (stepwise session calls, the captured-graph loop, and the forward-level entries) and checks
// they agree, plus the host-buffer op entries and the error statuses of the reference's
// EngineError variants.
//
//   iek_abi_test MODEL.gguf N_DECODE ID0 ID1 ...    (prompt token ids)
//
// Prints one JSON line {"tokens": [...], "first_logit": x, "checks": n} and exits 0, or prints the
// failed check and exits 1.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "iek.h"

static int g_checks = 0;

#define CHECK(cond, ...)                          \
  do {                                            \
    ++g_checks;                                   \
    if (!(cond)) {                                \
      fprintf(stderr, "check failed (%s:%d): ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);               \
      fprintf(stderr, " [last error: %s]\n", iek_last_error()); \
      exit(1);                                    \
    }                                             \
  } while (0)

#define OK(call) CHECK((call) == IEK_OK, "%s", #call)

int main(int argc, char** argv) {
  if (argc < 4) {
    fprintf(stderr, "usage: %s MODEL.gguf N_DECODE ID0 [ID1 ...]\n", argv[0]);
    return 2;
  }
  const char* path = argv[1];
  const int n_decode = atoi(argv[2]);
  std::vector<uint32_t> prompt;
  for (int i = 3; i < argc; ++i) prompt.push_back((uint32_t)strtoul(argv[i], nullptr, 10));

  // errors before anything loads
  iek_model* bad = nullptr;
  CHECK(iek_model_load("/nonexistent/model.gguf", 0, &bad) == IEK_ERR_MODEL, "missing file is a Model error");

  iek_model* model = nullptr;
  OK(iek_model_load(path, 0, &model));
  iek_model_config cfg;
  OK(iek_model_config_get(model, &cfg));
  CHECK(cfg.vocab_size > 0 && cfg.n_layers > 0 && cfg.hidden_dim > 0, "config");
  iek_load_timings lt;
  OK(iek_model_load_timings(model, &lt));
  CHECK(lt.tensor_load_ms >= 0 && lt.hbm_bytes > 0, "load timings");

  iek_session* s = nullptr;
  OK(iek_session_create(model, &s));

  // 1. stepwise: prefill, then { greedy_next_token; decode_token }
  OK(iek_session_prefill(s, prompt.data(), prompt.size()));
  std::vector<float> logits(cfg.vocab_size);
  OK(iek_session_logits_last_token(s, logits.data(), logits.size()));
  const float first_logit = logits[0];
  uint32_t want_first = 0;
  OK(iek_argmax(logits.data(), logits.size(), &want_first));  // host-buffer op on the session's logits
  std::vector<uint32_t> step_ids;
  for (int i = 0; i < n_decode; ++i) {
    uint32_t t = 0;
    OK(iek_greedy_next_token(s, &t));
    if (i == 0) CHECK(t == want_first, "greedy token %u != argmax of the logits %u", t, want_first);
    step_ids.push_back(t);
    OK(iek_session_decode_token(s, t));
  }
  uint64_t kv = 0;
  OK(iek_session_kv_len(s, &kv));
  CHECK(kv == prompt.size() + (size_t)n_decode, "kv_len %llu", (unsigned long long)kv);

  // 2. the captured-graph greedy loop from a fresh cache
  OK(iek_session_reset(s));
  OK(iek_session_prefill(s, prompt.data(), prompt.size()));
  std::vector<uint32_t> graph_ids(n_decode);
  OK(iek_session_generate_greedy(s, (size_t)n_decode, graph_ids.data()));
  for (int i = 0; i < n_decode; ++i)
    CHECK(graph_ids[i] == step_ids[i], "graph step %d: %u != %u", i, graph_ids[i], step_ids[i]);

  // 3. forward level: embed + prefill_forward, then embed(1) + decode_forward per token
  OK(iek_session_reset(s));
  OK(iek_session_embed(s, prompt.data(), prompt.size()));
  OK(iek_session_prefill_forward(s));
  for (int i = 0; i < n_decode; ++i) {
    uint32_t t = 0;
    OK(iek_greedy_next_token(s, &t));
    CHECK(t == step_ids[i], "forward-level step %d: %u != %u", i, t, step_ids[i]);
    OK(iek_session_embed(s, &t, 1));
    OK(iek_session_decode_forward(s));
  }

  // error statuses (src/error.rs:5-38)
  OK(iek_session_reset(s));
  CHECK(iek_session_prefill(s, prompt.data(), 0) == IEK_ERR_MODEL, "empty prompt");
  uint32_t oov = (uint32_t)cfg.vocab_size;
  CHECK(iek_session_prefill(s, &oov, 1) == IEK_ERR_MODEL, "out-of-vocabulary id");
  uint32_t tok = 0;
  CHECK(iek_greedy_next_token(s, &tok) == IEK_ERR_MODEL, "greedy on an empty state");
  OK(iek_session_prefill(s, prompt.data(), prompt.size()));
  std::vector<uint32_t> sink(cfg.context_length + 1);
  CHECK(iek_session_generate_greedy(s, cfg.context_length, sink.data()) == IEK_ERR_KV_CACHE, "KV cache full");

  // host-buffer ops: a known-answer F32 matmul in ggml layout (W(k, n) at k + n*K)
  {
    const float a[2 * 3] = {1, 2, 3, 4, 5, 6};
    const float w[3 * 2] = {1, 0, -1, 2, 1, 0};  // column n=0: (1, 0, -1); n=1: (2, 1, 0)
    iek_weight wt{IEK_F32, w, sizeof(w), 0};
    float out[4] = {0, 0, 0, 0};
    OK(iek_matmul(a, 2, 3, &wt, 2, out));
    CHECK(out[0] == -2 && out[1] == 4 && out[2] == -2 && out[3] == 13, "matmul %g %g %g %g", out[0], out[1], out[2],
          out[3]);
    wt.bytes = sizeof(w) - 4;
    CHECK(iek_matmul(a, 2, 3, &wt, 2, out) == IEK_ERR_MATMUL, "short weight buffer");
    float sm[3];
    const float x[3] = {0, 0, 0};
    OK(iek_softmax(x, sm, 3));
    CHECK(std::fabs(sm[1] - 1.0f / 3.0f) < 1e-7f, "softmax");
    CHECK(iek_softmax(x, sm, 0) == IEK_ERR_OP, "empty softmax");
    const float bad_logits[2] = {1.0f, NAN};
    CHECK(iek_argmax(bad_logits, 2, &tok) == IEK_ERR_SAMPLING, "non-finite logits");
  }

  iek_session_free(s);
  iek_model_free(model);
  printf("{\"tokens\": [");
  for (int i = 0; i < n_decode; ++i) printf("%s%u", i ? ", " : "", step_ids[i]);
  printf("], \"first_logit\": %.9g, \"checks\": %d}\n", first_logit, g_checks);
  return 0;
}
