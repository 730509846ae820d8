// Greedy generation through the C++ host API (include/grout.hpp), the shape
// of the reference's own token-driven callers (benchmarks/src/bin/
// grout_bench.rs): load, warmup, prefill a prompt of token ids, then greedy
// decode steps.
//
//   grout_generate <model dir or .gguf> <max_ctx> <n_decode> <token> [<token> ...]
//
// Prints, one item per line:
//   meta vocab=<V> max_ctx=<M> arch=<arch> eos=<id,id,...>
//   prefill_logits <the prompt's last-token logits, each as a hex float>
//   tokens <the prefill's greedy token, then one per decode step>
//   position <the position the next decode would write>
// Errors go to stderr with the ABI status code; the exit status is 1.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "grout.hpp"

namespace {

std::uint32_t argmax(const std::vector<float>& v) {
  std::size_t best = 0;  // first maximum, as the device argmax breaks ties
  for (std::size_t i = 1; i < v.size(); ++i)
    if (v[i] > v[best]) best = i;
  return static_cast<std::uint32_t>(best);
}

long parse_long(const char* s, const char* what) {
  char* end = nullptr;
  const long v = std::strtol(s, &end, 10);
  if (end == s || *end != '\0' || v < 0)
    throw grout::Error(GROUT_EINVAL, std::string("bad ") + what + ": " + s);
  return v;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 5) {
    std::fprintf(stderr, "usage: %s <model> <max_ctx> <n_decode> <token> [<token> ...]\n",
                 argv[0]);
    return 2;
  }
  try {
    grout::LoadOpts opts;
    opts.max_ctx = static_cast<std::size_t>(parse_long(argv[2], "max_ctx"));
    const long n_decode = parse_long(argv[3], "n_decode");
    std::vector<std::uint32_t> prompt;
    for (int i = 4; i < argc; ++i)
      prompt.push_back(static_cast<std::uint32_t>(parse_long(argv[i], "token")));

    grout::Engine eng = grout::Engine::load(argv[1], opts);
    const grout::ModelMeta& m = eng.meta();
    std::printf("meta vocab=%zu max_ctx=%zu arch=%s eos=", m.vocab_size, m.max_ctx,
                m.arch.c_str());
    for (std::size_t i = 0; i < m.eos_token_ids.size(); ++i)
      std::printf("%s%u", i ? "," : "", m.eos_token_ids[i]);
    std::printf("\n");

    eng.warmup();
    const grout::Logits logits = eng.prefill(prompt);
    std::printf("prefill_logits");
    for (float x : logits.as_slice()) std::printf(" %a", static_cast<double>(x));
    std::printf("\n");

    std::uint32_t tok = argmax(logits.values);
    std::printf("tokens %u", tok);
    for (long i = 0; i < n_decode; ++i) {
      tok = eng.decode_greedy(tok);
      std::printf(" %u", tok);
    }
    std::printf("\nposition %zu\n", eng.position());
    return 0;
  } catch (const grout::Error& e) {
    std::fprintf(stderr, "grout error %d: %s\n", e.code(), e.what());
    return 1;
  }
}
