// tests/cpp/test_profiler.cpp -- the profiler's arithmetic and the residency
// pass-through, on the CPU.  The device backend takes plain offsets, so every
// device-domain rule (self time of nested spans, idle between outermost spans
// per stream, floors, dropped spans) is checked on synthetic spans with exact
// expected values, read back through the CSV and JSON writers.  The rules are
// the ones the reference's profiler states (/root/reference/src/profiler/
// profiler.h:1-139) and its unit test grades (tests/unit/test_c21_profiler.cpp).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "../../include/knj/profiler.h"
#include "../../include/knj/residency.h"

namespace {

int g_fail = 0, g_checks = 0;
#define EXPECT(x)                                                   \
  do {                                                              \
    ++g_checks;                                                     \
    if (!(x)) {                                                     \
      ++g_fail;                                                     \
      std::printf("FAIL %s:%d  %s\n", __FILE__, __LINE__, #x);      \
    }                                                               \
  } while (0)

std::string capture(void (knj::Profiler::*w)(std::FILE*) const) {
  std::FILE* f = std::tmpfile();
  (knj::Profiler::get().*w)(f);
  std::rewind(f);
  std::string s;
  char buf[4096];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) s.append(buf, n);
  std::fclose(f);
  return s;
}

struct Csv {
  bool found = false;
  unsigned long long ops = 0, dev = 0, idle = 0, host = 0;
  std::string clock;
};

Csv csv(const char* comp) {
  const std::string s = capture(&knj::Profiler::report_csv);
  Csv r;
  size_t p = 0;
  while (p < s.size()) {
    size_t e = s.find('\n', p);
    if (e == std::string::npos) e = s.size();
    const std::string line = s.substr(p, e - p);
    p = e + 1;
    const size_t c = line.find(',');
    if (c == std::string::npos || line.substr(0, c) != comp) continue;
    char clock[32] = {0};
    if (std::sscanf(line.c_str() + c + 1, "%llu,%llu,%llu,%llu,%31[^,]", &r.ops, &r.dev, &r.idle,
                    &r.host, clock) == 5) {
      r.found = true;
      r.clock = clock;
    }
  }
  return r;
}

double json_self(const char* comp) {
  const std::string s = capture(&knj::Profiler::report_json);
  const size_t at = s.find(std::string("\"component\": \"") + comp + "\"");
  if (at == std::string::npos) return -1;
  const size_t v = s.find("\"dev_ns_self\": ", at);
  return std::atof(s.c_str() + v + 15);
}

void arm(bool subtract, const char* detail = "class", int warmup = 0) {
  knj::ProfileConfig pc;
  pc.on = true;
  pc.format = "csv";
  pc.detail = detail;
  pc.floor_ops = 0;
  pc.warmup_steps = warmup;
  pc.subtract_floor = subtract;
  knj::Profiler::get().configure(pc);
}

}  // namespace

int main(int argc, char** argv) {
  knj::Profiler& p = knj::Profiler::get();

  // host domain: dev == host; a gap between outer ops is idle of the next op
  arm(false);
  p.begin("a");
  p.end();
  const auto t0 = std::chrono::steady_clock::now();
  while (std::chrono::steady_clock::now() - t0 < std::chrono::milliseconds(3))
    std::this_thread::sleep_for(std::chrono::microseconds(200));
  p.begin("b");
  p.begin("b-inner:1");
  p.end();
  p.end();
  Csv a = csv("a"), b = csv("b"), bi = csv("b-inner");
  EXPECT(a.found && b.found && bi.found);
  EXPECT(a.dev == a.host && b.dev == b.host && a.clock == "host");
  EXPECT(a.idle == 0 && b.idle >= 2500000ull && bi.idle == 0);
  EXPECT(p.nested_ops() == 1 && p.max_depth() == 2);

  // device backend: host markers stop writing dev
  arm(false);
  p.enable_device_backend();
  p.begin("g");
  p.end();
  Csv g = csv("g");
  EXPECT(g.found && g.host > 0 && g.dev == 0 && g.idle == 0 && g.clock == "device");

  // device spans: nesting by containment, idle between outermost spans, per stream
  //   stream 0: p [100,900] with c1 [200,300] and c2 [400,700] (c2 holds c3 [500,600]),
  //             then q [1000,1300] and r [1300,1400] back to back
  //   stream 2: s [50,150], t [450,500]
  p.device_span("q", 1000, 1300, 0);  // out of order on purpose
  p.device_span("p", 100, 900, 0);
  p.device_span("c1", 200, 300, 0);
  p.device_span("c2", 400, 700, 0);
  p.device_span("c3", 500, 600, 0);
  p.device_span("r", 1300, 1400, 0);
  p.device_span("s", 50, 150, 2);
  p.device_span("t", 450, 500, 2);
  Csv P = csv("p"), C1 = csv("c1"), C2 = csv("c2"), C3 = csv("c3"), Q = csv("q"), R = csv("r");
  Csv S = csv("s"), T = csv("t");
  EXPECT(P.dev == 800 - 100 - 300);  // children c1 (100) and c2 (300)
  EXPECT(C1.dev == 100 && C2.dev == 200 && C3.dev == 100);
  EXPECT(P.dev + C1.dev + C2.dev + C3.dev == 800);
  EXPECT(Q.dev == 300 && Q.idle == 100);  // 1000 - 900
  EXPECT(R.dev == 100 && R.idle == 0);
  EXPECT(P.idle == 0 && C1.idle == 0 && C3.idle == 0);
  EXPECT(S.dev == 100 && S.idle == 0 && T.dev == 50 && T.idle == 300);
  EXPECT(p.device_spans() == 8);

  // equal starts: the longer span is the parent
  arm(false);
  p.enable_device_backend();
  p.device_span("inner", 0, 100, 0);
  p.device_span("outer", 0, 400, 0);
  EXPECT(csv("outer").dev == 300 && csv("inner").dev == 100);

  // device floor: raw until measured; then per span for a device-only row and
  // per op for a row with host markers, never below zero
  arm(true);
  p.enable_device_backend();
  p.device_span("k", 0, 1000, 0);
  p.device_span("k", 2000, 2600, 0);
  p.device_span("tiny", 3000, 3010, 0);
  p.begin("m");
  p.end();
  p.device_span("m", 4000, 5000, 0);
  EXPECT(json_self("k") == 1600.0);
  p.set_device_floor(250, 64);
  EXPECT(json_self("k") == 1600.0 - 2 * 250);
  EXPECT(json_self("tiny") == 0.0);
  EXPECT(json_self("m") == 1000.0 - 250);
  EXPECT(csv("k").dev == 1600);  // the CSV keeps the raw measurement

  // dropped spans are stated
  p.set_device_dropped(5);
  const std::string table = capture(&knj::Profiler::report_table);
  EXPECT(table.find("5 dropped") != std::string::npos);
  EXPECT(table.find("device floor: 0.250 us") != std::string::npos);

  // detail levels
  arm(false, "layer");
  p.enable_device_backend();
  p.device_span("qkv:3:k_gemv_q4k", 0, 10, 0);
  p.device_span("qkv:4:k_gemv_q4k", 10, 30, 0);
  EXPECT(csv("qkv:3").dev == 10 && csv("qkv:4").dev == 20 && !csv("qkv").found);
  arm(false, "class");
  p.enable_device_backend();
  p.device_span("qkv:3:k_gemv_q4k", 0, 10, 0);
  p.device_span("qkv:4:k_gemv_q4k", 10, 30, 0);
  EXPECT(csv("qkv").dev == 30);
  arm(false, "kernel");
  p.enable_device_backend();
  p.device_span("qkv:3:k_gemv_q4k", 0, 10, 0);
  EXPECT(csv("qkv:3:k_gemv_q4k").dev == 10);

  // warmup: ops of the first steps are discarded
  arm(false, "class", 2);
  for (int s = 0; s < 5; ++s) {
    p.begin("step");
    p.end();
    p.step_done();
  }
  EXPECT(csv("step").ops == 3 && p.steps_kept() == 3 && p.steps_discarded() == 2);

  // the host floor goes through the same path and leaves no row behind
  knj::ProfileConfig pc;
  pc.on = true;
  pc.floor_ops = 64;
  pc.warmup_steps = 0;
  p.configure(pc);
  p.measure_floor();
  EXPECT(p.floor_n() == 64 && p.floor_host_ns() > 0 && p.op_count() == 0);
  EXPECT(capture(&knj::Profiler::report_csv).find("__floor") == std::string::npos);

  // an outer marker left open across step boundaries: its children are
  // settled with it, not before (self time of the outer = span - children)
  arm(false, "class", 0);
  p.begin("outer");
  for (int s = 0; s < 3; ++s) {
    p.begin("inner");
    const auto w0 = std::chrono::steady_clock::now();
    while (std::chrono::steady_clock::now() - w0 < std::chrono::microseconds(300)) {
    }
    p.end();
    p.step_done();
  }
  p.end();
  p.step_done();
  {
    Csv o = csv("outer"), in = csv("inner");
    EXPECT(o.found && in.found && o.ops == 1 && in.ops == 3);
    EXPECT(in.host >= 900000ull && o.host < in.host);
    EXPECT(in.idle == 0);  // nested: gaps inside an open marker are not idle
  }

  // idle across settled steps: the gap between the last op of one step and
  // the first of the next is charged even though a step boundary settled the log
  arm(false, "class", 0);
  p.begin("x");
  p.end();
  p.step_done();
  {
    const auto w0 = std::chrono::steady_clock::now();
    while (std::chrono::steady_clock::now() - w0 < std::chrono::milliseconds(1)) {
    }
  }
  p.begin("y");
  p.end();
  p.step_done();
  EXPECT(csv("y").idle >= 900000ull && csv("x").idle == 0);

  // files: profile.{txt,json,csv} in the directory given on the command line
  if (argc > 1) {
    knj::ProfileConfig fc;
    fc.on = true;
    fc.floor_ops = 16;
    fc.warmup_steps = 0;
    fc.dir = argv[1];
    p.configure(fc);
    p.enable_device_backend();
    p.set_device_floor(100, 8);
    p.device_span("head:0:k", 0, 1000, 0);
    p.device_span("qkv:1:k", 1500, 2000, 0);
    p.begin("decode");
    p.end();
    knj::ResidencyStats rs;
    rs.measured = true;
    rs.vram_pct = 100.0;
    p.note_residency(rs);
    EXPECT(p.write_dir() == 3);
  }

  // off: nothing is recorded
  knj::ProfileConfig off;
  p.configure(off);
  p.begin("never");
  p.end();
  p.device_span("never-dev", 0, 5, 0);
  EXPECT(!csv("never").found && !csv("never-dev").found);
  EXPECT(capture(&knj::Profiler::report_table).find("profile: off") != std::string::npos);

  // residency pass-through: everything pinned in VRAM, nothing evictable
  knj::ResidencyManager res(48, 128, 4096, 256);
  EXPECT(res.n_experts() == 48u * 128u && res.n_kv_pages() == 48u * 16u);
  EXPECT(res.locate(knj::ExpertId{47, 127}) == knj::Residency::PINNED);
  EXPECT(res.locate(knj::ExpertId{48, 0}) == knj::Residency::ABSENT);
  EXPECT(res.demand_or_fallback(knj::ExpertId{3, 9}));
  EXPECT(!res.demand(knj::ExpertId{3, 128}, knj::KVTier::VRAM));
  res.demote(knj::ExpertId{1, 1});
  res.demote_kv(knj::KvPageId{1, 2});
  EXPECT(res.refused_demotions() == 2 && res.eviction_candidates().empty());
  EXPECT(res.kernel_view().ready_kv(knj::KvPageId{0, 15}) && !res.ready_kv(knj::KvPageId{0, 16}));
  res.begin_layer(5);
  res.tick();
  EXPECT(res.tick_index() == 1 && res.layer() == 5);
  const knj::ResidencyStats st = res.stats();
  EXPECT(st.measured && st.vram_pct == 100.0 && st.slots_used == 48u * 128u &&
         st.slots_total == st.slots_used && st.evictions == 0 && st.prefetch_hit == 0.5);
  EXPECT(std::strcmp(knj::to_string(knj::Residency::PINNED), "PINNED") == 0);

  std::printf("profiler/residency: %d checks, %d failed\n", g_checks, g_fail);
  return g_fail ? 1 : 0;
}
