// kanjoos_amd/host/kanjoos_run.cpp -- command-line driver of the device decode step.
//
// The shape of the reference's kanjoos-run prefill -> greedy decode loop and its
// --bench PP TG mode (/root/reference/src/cli/main.cpp:245-279, 451-568), over
// the C++ Model class; weights come from a qwen3moe GGUF file (--model) or are
// the seeded synthetic Qwen3-30B-A3B-shaped model.
//
//   kanjoos-run [--layers N] [--ctx N] [--seed S] [--prompt N] [--n-predict N]
//               [--bench PP TG] [--small] [--model PATH.gguf] [--fill-kv N]
//               [--profiling[=table|json|csv|no-subtract|off]] [--profile-dir DIR]
//               [--profile-floor N] [--profile-warmup N] [--profile-detail=class|layer|kernel]
//
// --bench PP runs the PP tokens as one forward call (the prompt pass, as the
// reference's normal mode runs a prompt, main.cpp:521-528); the reference's
// --bench feeds them one call each (main.cpp:255-257), which KNJ_PROMPT_STEPS=1
// reproduces here.
//
// --profiling (main.cpp:47-56, 94-98, 198-223, 314-318) times the decode with
// a dispatch event pair around every kernel launch (Model::decode_greedy_profiled)
// and prints the profiler's report before the token line; the tokens are the
// same as without it.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../../include/knj/backend.h"
#include "../../include/knj/model.h"
#include "../../include/knj/profiler.h"
#include "../../include/knj/residency.h"

int main(int argc, char** argv) {
  int layers = 48, ctx = 4352, prompt = 16, n_predict = 32, pp = 0, tg = 0, fill_kv = 0;
  uint64_t seed = 0;
  bool small = false;
  std::string model_path;  // --model PATH: a qwen3moe GGUF instead of synthetic weights
  knj::ProfileConfig pc;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&](const char* name) {
      if (i + 1 >= argc) {
        std::fprintf(stderr, "%s needs a value\n", name);
        std::exit(2);
      }
      return std::atoi(argv[++i]);
    };
    if (a == "--layers") layers = next("--layers");
    else if (a == "--ctx") ctx = next("--ctx");
    else if (a == "--seed") seed = (uint64_t)next("--seed");
    else if (a == "--prompt") prompt = next("--prompt");
    else if (a == "--n-predict") n_predict = next("--n-predict");
    else if (a == "--fill-kv") fill_kv = next("--fill-kv");
    else if (a == "--small") small = true;
    else if (a == "--model") {
      if (i + 1 >= argc) {
        std::fprintf(stderr, "--model needs a value\n");
        return 2;
      }
      model_path = argv[++i];
    }
    else if (a == "--profile-dir") {
      if (i + 1 >= argc) {
        std::fprintf(stderr, "--profile-dir needs a value\n");
        return 2;
      }
      pc.dir = argv[++i];
    } else if (a == "--profile-floor") pc.floor_ops = next("--profile-floor");
    else if (a == "--profile-warmup") pc.warmup_steps = next("--profile-warmup");
    else if (a.rfind("--profile-detail=", 0) == 0) {
      pc.detail = a.substr(17);
      if (pc.detail != "class" && pc.detail != "layer" && pc.detail != "kernel") {
        std::fprintf(stderr, "--profile-detail must be class, layer or kernel\n");
        return 2;
      }
    } else if (a == "--profiling" || a.rfind("--profiling=", 0) == 0) {
      const std::string fmt = a.size() > 12 ? a.substr(12) : "table";
      pc.on = fmt != "off";
      pc.format = "table";
      if (fmt == "no-subtract") pc.subtract_floor = false;
      else if (fmt == "json" || fmt == "csv") pc.format = fmt;
      else if (fmt != "table" && fmt != "off") {
        std::fprintf(stderr, "--profiling=%s: expected off|table|json|csv|no-subtract\n", fmt.c_str());
        return 2;
      }
    } else if (a == "--bench") {
      pp = next("--bench");
      tg = next("--bench");
    } else {
      std::fprintf(stderr, "unknown argument %s\n", a.c_str());
      return 2;
    }
  }
  if (!model_path.empty()) {  // refuse a bad file before touching the device
    knj_model_config probe{};
    if (knj_gguf_probe(model_path.c_str(), ctx, &probe) != 0) {
      std::fprintf(stderr, "model: %s\n", knj_last_error());
      return 3;
    }
  }
  auto backend = knj::Backend::create();
  if (!backend) {
    std::fprintf(stderr, "device refused: %s\n", knj::Backend::knj_last_refusal());
    return 6;
  }
  knj_model_config c{};
  c.n_layer = layers; c.n_embd = 2048; c.n_head = 32; c.n_head_kv = 4; c.head_dim = 128;
  c.n_ff = 768; c.n_expert = 128; c.n_expert_used = 8; c.n_vocab = 151936; c.n_ctx = ctx;
  c.rms_eps = 1e-6f; c.rope_base = 1e6f; c.type_embd = KNJ_TYPE_BF16; c.type_attn = KNJ_TYPE_Q4_K;
  c.type_gate_up = KNJ_TYPE_Q4_K; c.type_down = KNJ_TYPE_Q4_K; c.type_head = KNJ_TYPE_BF16;
  c.init_std = 0.02f;
  if (small) {
    c.n_embd = 512; c.n_head = 8; c.n_head_kv = 2; c.head_dim = 64; c.n_ff = 256;
    c.n_expert = 16; c.n_expert_used = 4; c.n_vocab = 4096;
  }
  try {
    knj::Model::Options opt;
    opt.n_ctx = ctx;
    auto m = model_path.empty() ? knj::Model::open_synthetic(c, seed, opt)
                                : knj::Model::open(model_path, opt);
    c.n_vocab = m->geom().n_vocab;
    std::printf("%s\n", m->geom().describe().c_str());
    std::mt19937 rng((uint32_t)seed);
    auto run_prompt = [&](int n) {
      std::vector<int32_t> toks((size_t)n);
      for (auto& t : toks) t = (int32_t)(rng() % (uint32_t)c.n_vocab);
      const float* lg = m->forward(toks.data(), n);
      int best = 0;
      for (int v = 1; v < c.n_vocab; ++v)
        if (lg[v] > lg[best]) best = v;  // first maximum wins (main.cpp:126-132)
      return best;
    };
    using clk = std::chrono::steady_clock;
    if (pp > 0 || tg > 0) {
      const auto t0 = clk::now();
      const int first = run_prompt(pp > 0 ? pp : 1);
      const auto t1 = clk::now();
      const auto out = m->decode_greedy(first, tg > 0 ? tg : 1);
      const auto t2 = clk::now();
      const double pp_s = std::chrono::duration<double>(t1 - t0).count();
      const double tg_s = std::chrono::duration<double>(t2 - t1).count();
      std::printf("bench: pp %d tokens %.1f tok/s, tg %d tokens %.1f tok/s (%.3f ms/token)\n", pp,
                  pp / pp_s, tg, tg / tg_s, 1000.0 * tg_s / tg);
      (void)out;
      return 0;
    }
    // --fill-kv N: start from a seeded N-token context (the decode benchmarks'
    // long-context state) instead of position 0
    if (fill_kv > 0) m->fill_kv(fill_kv, seed);
    knj::Profiler& prof = knj::Profiler::get();
    prof.configure(pc);
    if (pc.on) {
      prof.enable_device_backend();
      uint64_t floor_ns = 0;
      const int floor_n = pc.floor_ops > 0 ? std::min(pc.floor_ops, 4096) : 0;
      if (floor_n > 0 && knj_device_floor(floor_n, &floor_ns) == KNJ_OK)
        prof.set_device_floor(floor_ns, floor_n);
      prof.measure_floor();
    }
    int first = 0;
    {
      KNJ_PROFILE_OP("prefill");
      first = run_prompt(prompt);
    }
    std::vector<int32_t> out;
    {
      KNJ_PROFILE_OP("decode");
      out = pc.on ? m->decode_greedy_profiled(first, n_predict, prof)
                  : m->decode_greedy(first, n_predict);
    }
    if (pc.on) {
      const knj::ModelGeometry& g = m->geom();
      knj::ResidencyManager res((uint32_t)g.n_layer, (uint32_t)g.n_expert, (uint32_t)m->n_ctx(), 256);
      prof.note_residency(res.stats());
      prof.note_transfer(m->transfer_stats());
      prof.print_header(stdout, "0.1", "gfx950", g.describe());
      prof.report(stdout);
      prof.write_dir();
    }
    std::printf("tokens:");
    for (int32_t t : out) std::printf(" %d", t);
    std::printf("\n");
  } catch (const std::exception& e) {
    std::fprintf(stderr, "%s\n", e.what());
    return 9;
  }
  return 0;
}
