// kanjoos_amd/host/knj_profiler.cpp -- the profiler of include/knj/profiler.h.
//
// Design: an interval log and one sweep.
//  * A host marker pair, once closed, and a device span are both an
//    Interval {component, lane, source, t0, t1}.  Closing a marker does no
//    arithmetic beyond logging; nesting is not tracked while the step runs.
//  * settle() sorts the log by (source, lane, start, longer first, begin
//    order) and walks each lane with a containment stack: an interval that
//    starts before the innermost open one ends is its child, so the parent's
//    self time loses the overlap; an interval with nothing open is outermost,
//    and its distance from the previous outermost end on the lane is its idle.
//    Host markers and device spans therefore follow one rule.
//  * The lane edges (last outermost end per lane) outlive a sweep, so the log
//    can be settled at every step boundary and stays small.
//  * The host floor is timed on a private Profiler instance through the same
//    begin/end path, so this instance's state is never touched.
// The CSV columns and JSON keys are the reference's file format
// (/root/reference/src/profiler/profiler.h:44-175 describes them), so readers
// of its profile files read these.
#include "../../include/knj/profiler.h"

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cstring>
#include <sys/stat.h>

namespace knj {
namespace {

uint64_t clock_ns() {
  using namespace std::chrono;
  return (uint64_t)duration_cast<nanoseconds>(steady_clock::now().time_since_epoch()).count();
}

// Peak resident set of this process in MiB (VmHWM), 0 when unreadable.
double peak_rss_mib() {
  std::FILE* f = std::fopen("/proc/self/status", "r");
  if (!f) return 0.0;
  char line[256];
  double kib = 0.0;
  while (std::fgets(line, sizeof(line), f))
    if (std::strncmp(line, "VmHWM:", 6) == 0) kib = std::atof(line + 6);
  std::fclose(f);
  return kib / 1024.0;
}

// The part of `name` kept at a detail level: the first `fields` ':'-separated
// fields (all of them when fields <= 0 or the name has fewer).
std::string leading_fields(const char* name, int fields) {
  const char* s = name ? name : "";
  if (fields <= 0) return s;
  const char* p = s;
  for (int seen = 0; *p; ++p)
    if (*p == ':' && ++seen == fields) break;
  return std::string(s, (size_t)(p - s));
}

// Minimal streaming JSON object writer: commas and quoting are its business.
class Json {
 public:
  explicit Json(std::FILE* f) : f_(f) {}
  void open(const char* key, char bracket) {
    sep(key);
    std::fputc(bracket, f_);
    first_ = true;
    ++depth_;
  }
  void close(char bracket) {
    --depth_;
    std::fputc('\n', f_);
    indent();
    std::fputc(bracket, f_);
    first_ = false;
  }
  void str(const char* key, const std::string& v) {
    sep(key);
    quoted(v);
  }
  void u64(const char* key, uint64_t v) {
    sep(key);
    std::fprintf(f_, "%llu", (unsigned long long)v);
  }
  void i32(const char* key, int v) {
    sep(key);
    std::fprintf(f_, "%d", v);
  }
  void num(const char* key, double v, int prec) {
    sep(key);
    std::fprintf(f_, "%.*f", prec, v);
  }
  void flag(const char* key, bool v) {
    sep(key);
    std::fputs(v ? "true" : "false", f_);
  }
  // a one-line object inside an array or as a value
  void inline_open(const char* key) {
    sep(key);
    std::fputc('{', f_);
    inline_first_ = true;
    inline_ = true;
  }
  void inline_close() {
    std::fputc('}', f_);
    inline_ = false;
  }

 private:
  void indent() {
    for (int i = 0; i < depth_; ++i) std::fputs("  ", f_);
  }
  void quoted(const std::string& v) {
    std::fputc('"', f_);
    for (char c : v) {
      if (c == '"' || c == '\\') std::fputc('\\', f_);
      if (c == '\n') {
        std::fputs("\\n", f_);
        continue;
      }
      std::fputc(c, f_);
    }
    std::fputc('"', f_);
  }
  void sep(const char* key) {
    if (inline_) {
      if (!inline_first_) std::fputs(", ", f_);
      inline_first_ = false;
    } else {
      if (!first_) std::fputc(',', f_);
      if (depth_ > 0) std::fputc('\n', f_);
      indent();
      first_ = false;
    }
    if (key) {
      quoted(key);
      std::fputs(": ", f_);
    }
  }
  std::FILE* f_;
  int depth_ = 0;
  bool first_ = true, inline_ = false, inline_first_ = true;
};

}  // namespace

const char* clock_domain_name(ClockDomain d) {
  switch (d) {
    case ClockDomain::Host: return "host";
    case ClockDomain::Device: return "device";
    default: return "none";
  }
}

Profiler& Profiler::get() {
  static Profiler instance;
  return instance;
}

// A new configuration starts a new session: no device backend until one is
// attached again, host clock when on.
void Profiler::configure(const ProfileConfig& c) {
  opts_ = c;
  dev_ = DeviceInfo{};
  domain_ = opts_.on ? ClockDomain::Host : ClockDomain::None;
  reset();
}

void Profiler::reset() {
  names_.clear();
  ids_.clear();
  tally_.clear();
  log_.clear();
  open_.clear();
  for (auto& src : edge_)
    for (auto& e : src) e = LaneEdge{};
  count_ = Counters{};
  dev_.recorded = dev_.dropped = 0;
}

void Profiler::enable_device_backend() {
  dev_.enabled = true;
  domain_ = ClockDomain::Device;
}

void Profiler::set_device_floor(uint64_t ns, int n) {
  dev_.floor_ns = ns;
  dev_.floor_n = n;
  dev_.floor_known = true;
}

uint32_t Profiler::component(const char* name) const {
  const int fields = opts_.detail == "class" ? 1 : opts_.detail == "layer" ? 2 : 0;
  std::string key = leading_fields(name, fields);
  auto it = ids_.find(key);
  if (it != ids_.end()) return it->second;
  const uint32_t id = (uint32_t)names_.size();
  names_.push_back(key);
  tally_.emplace_back();
  ids_.emplace(std::move(key), id);
  return id;
}

void Profiler::begin(const char* name, int stream) {
  if (!opts_.on) return;
  if (open_.empty()) {
    open_lane_ = (uint8_t)(stream >= 0 && stream < kLanes ? stream : 0);
  } else {
    ++count_.nested;
  }
  const uint32_t comp = component(name);
  open_.push_back(OpenMarker{comp, clock_ns(), count_.seq++});
  count_.depth = std::max<uint64_t>(count_.depth, open_.size());
}

void Profiler::end() {
  if (!opts_.on || open_.empty()) return;
  const uint64_t t1 = clock_ns();
  const OpenMarker m = open_.back();
  open_.pop_back();
  const bool counted = count_.steps >= (uint64_t)opts_.warmup_steps;
  log_.push_back(Interval{m.comp, open_lane_, Source::Host, counted, m.t0, std::max(t1, m.t0), m.seq});
  if (counted) ++count_.ops;
}

void Profiler::step_done() {
  if (!opts_.on) return;
  if (count_.steps < (uint64_t)opts_.warmup_steps)
    ++count_.discarded;
  else
    ++count_.kept;
  ++count_.steps;
  if (open_.empty()) settle();
}

void Profiler::device_span(const char* name, uint64_t start_ns, uint64_t end_ns, int stream) {
  if (!opts_.on || !dev_.enabled) return;
  const uint8_t lane = (uint8_t)(stream >= 0 && stream < kLanes ? stream : 0);
  log_.push_back(Interval{component(name), lane, Source::Device, true, start_ns,
                          std::max(start_ns, end_ns), count_.seq++});
  ++dev_.recorded;
}

void Profiler::settle() const {
  // Host intervals wait while a marker is open: their parent is not logged yet.
  const bool host_ready = open_.empty();
  auto ready = [&](const Interval& iv) { return iv.src == Source::Device || host_ready; };
  auto split = std::stable_partition(log_.begin(), log_.end(), ready);
  std::vector<Interval> todo(log_.begin(), split);
  log_.erase(log_.begin(), split);
  std::sort(todo.begin(), todo.end(), [](const Interval& a, const Interval& b) {
    if (a.src != b.src) return a.src < b.src;
    if (a.lane != b.lane) return a.lane < b.lane;
    if (a.t0 != b.t0) return a.t0 < b.t0;
    if (a.t1 != b.t1) return a.t1 > b.t1;
    return a.seq < b.seq;
  });
  struct Frame {
    const Interval* iv;
    uint64_t covered;  // time taken by children
  };
  std::vector<Frame> stack;
  auto retire = [&]() {
    const Frame fr = stack.back();
    stack.pop_back();
    const Interval& iv = *fr.iv;
    const uint64_t len = iv.t1 - iv.t0;
    const uint64_t self = len > fr.covered ? len - fr.covered : 0;
    if (!iv.counted) return;
    Tally& t = tally_[iv.comp];
    if (iv.src == Source::Device) {
      t.dev_self += self;
    } else {
      t.host_self += self;
      if (!dev_.enabled) t.dev_self += self;  // host domain: one interval, both columns
    }
  };
  for (size_t i = 0; i < todo.size(); ++i) {
    const Interval& iv = todo[i];
    if (i > 0 && (todo[i - 1].src != iv.src || todo[i - 1].lane != iv.lane))
      while (!stack.empty()) retire();
    while (!stack.empty() && iv.t0 >= stack.back().iv->t1) retire();
    if (stack.empty()) {
      LaneEdge& e = edge_[(int)iv.src][iv.lane];
      const bool idle_applies = iv.src == Source::Device || !dev_.enabled;
      if (iv.counted && idle_applies && e.any && iv.t0 > e.last_end)
        tally_[iv.comp].idle += iv.t0 - e.last_end;
      e.last_end = e.any ? std::max(e.last_end, iv.t1) : iv.t1;
      e.any = true;
    } else {
      Frame& parent = stack.back();
      parent.covered += std::min(iv.t1, parent.iv->t1) - iv.t0;
    }
    if (iv.counted) {
      Tally& t = tally_[iv.comp];
      if (iv.src == Source::Device)
        ++t.spans;
      else
        ++t.ops;
    }
    stack.push_back(Frame{&iv, 0});
  }
  while (!stack.empty()) retire();
}

void Profiler::measure_floor() {
  host_floor_ = HostFloor{};
  const int n = std::max(0, opts_.floor_ops);
  if (n == 0) return;
  // A scratch instance runs the identical marker path; nothing of this one changes.
  Profiler probe;
  probe.opts_.on = true;
  probe.opts_.detail = "kernel";
  probe.opts_.warmup_steps = 0;
  probe.log_.reserve((size_t)n + 64);
  for (int i = 0; i < 64; ++i) {
    probe.begin("floor");
    probe.end();
  }
  const uint64_t t0 = clock_ns();
  for (int i = 0; i < n; ++i) {
    probe.begin("floor");
    probe.end();
  }
  const uint64_t t1 = clock_ns();
  host_floor_.n = n;
  host_floor_.ns = (t1 - t0) / (uint64_t)n;
}

std::vector<uint32_t> Profiler::by_dev_time() const {
  settle();
  std::vector<uint32_t> ids;
  for (uint32_t i = 0; i < (uint32_t)tally_.size(); ++i)
    if (tally_[i].ops || tally_[i].spans) ids.push_back(i);
  std::sort(ids.begin(), ids.end(), [&](uint32_t a, uint32_t b) {
    if (tally_[a].dev_self != tally_[b].dev_self) return tally_[a].dev_self > tally_[b].dev_self;
    return names_[a] < names_[b];
  });
  return ids;
}

// Floors come off per measurement and never below zero.  Device time takes the
// device floor only once one was measured (a host floor is never subtracted
// from device time); a component measured only by spans counts its spans.
double Profiler::dev_floor_of(const Tally& t) const {
  if (!opts_.subtract_floor) return 0.0;
  double per, n;
  if (dev_.enabled) {
    if (!dev_.floor_known) return 0.0;
    per = (double)dev_.floor_ns;
    n = (double)(t.ops ? t.ops : t.spans);
  } else {
    per = (double)host_floor_.ns;
    n = (double)t.ops;
  }
  return std::min(per * n, (double)t.dev_self);
}

double Profiler::host_floor_of(const Tally& t) const {
  if (!opts_.subtract_floor) return 0.0;
  return std::min((double)host_floor_.ns * (double)t.ops, (double)t.host_self);
}

void Profiler::print_header(std::FILE* f, const std::string& version, const std::string& device_line,
                            const std::string& budgets_line) const {
  std::fprintf(f, "\n  kanjoos-amd %s   device %s\n", version.c_str(), device_line.c_str());
  if (!budgets_line.empty()) std::fprintf(f, "    %s\n", budgets_line.c_str());
  std::fprintf(f,
               "    clock %s; rows are self time (max depth %llu); steps kept %llu, discarded "
               "%llu (warmup %d); %llu host op(s); peak rss %.0f MiB\n",
               clock_domain_name(domain_), (unsigned long long)count_.depth,
               (unsigned long long)count_.kept, (unsigned long long)count_.discarded,
               opts_.warmup_steps, (unsigned long long)count_.ops, peak_rss_mib());
  std::fprintf(f, "    profiling measures the run; it does not change what the step computes\n");
}

void Profiler::report_table(std::FILE* f) const {
  if (!opts_.on) {
    std::fprintf(f, "\nprofile: off\n");
    return;
  }
  const std::vector<uint32_t> ids = by_dev_time();
  double sum_dev = 0, sum_idle = 0, sum_host = 0;
  size_t width = 20;
  for (uint32_t i : ids) {
    sum_dev += (double)tally_[i].dev_self - dev_floor_of(tally_[i]);
    sum_idle += (double)tally_[i].idle;
    sum_host += (double)tally_[i].host_self - host_floor_of(tally_[i]);
    width = std::max(width, names_[i].size());
  }
  const int w = (int)width;
  std::fprintf(f, "\n  %-*s %7s %8s %7s %12s %12s %12s\n", w, "component", "ops", "spans", "%dev",
               "dev us", "idle us", "host us");
  for (uint32_t i : ids) {
    const Tally& t = tally_[i];
    const double dev = (double)t.dev_self - dev_floor_of(t);
    std::fprintf(f, "  %-*s %7llu %8llu %6.1f%% %12.2f %12.2f %12.2f\n", w, names_[i].c_str(),
                 (unsigned long long)t.ops, (unsigned long long)t.spans,
                 sum_dev > 0 ? 100.0 * dev / sum_dev : 0.0, dev / 1e3, (double)t.idle / 1e3,
                 ((double)t.host_self - host_floor_of(t)) / 1e3);
  }
  std::fprintf(f, "  total: dev %.2f us, idle %.2f us, host %.2f us\n", sum_dev / 1e3,
               sum_idle / 1e3, sum_host / 1e3);
  const char* sub = opts_.subtract_floor ? ", subtracted" : ", not subtracted (no-subtract)";
  if (host_floor_.n > 0)
    std::fprintf(f, "  host floor: %.3f us per marker pair (%d timed)%s\n",
                 (double)host_floor_.ns / 1e3, host_floor_.n, sub);
  else
    std::fprintf(f, "  host floor: not measured\n");
  std::fprintf(f, "  clock domain: %s%s\n", clock_domain_name(domain_),
               domain_ == ClockDomain::Host ? " (dev and host are the same host interval)" : "");
  if (dev_.enabled) {
    std::fprintf(f, "  device spans: %llu recorded, %llu dropped%s\n",
                 (unsigned long long)dev_.recorded, (unsigned long long)dev_.dropped,
                 dev_.dropped ? " -- the dev total is short by the dropped spans" : "");
    if (dev_.floor_known)
      std::fprintf(f, "  device floor: %.3f us per span (%d empty kernels)%s\n",
                   (double)dev_.floor_ns / 1e3, dev_.floor_n, sub);
    else
      std::fprintf(f, "  device floor: not measured -- dev rows are raw\n");
    std::fprintf(f, "  device resolution: event times are float ms; sub-0.1 us differences are "
                    "noise\n");
  }
  if (res_.measured)
    std::fprintf(f,
                 "  residency: vram %.1f%% ram %.1f%% nvme %.1f%%, slots %llu/%llu, evictions "
                 "%llu, prefetch hit %.2f, stall %.2f ms\n",
                 res_.vram_pct, res_.ram_pct, res_.nvme_pct, (unsigned long long)res_.slots_used,
                 (unsigned long long)res_.slots_total, (unsigned long long)res_.evictions,
                 res_.prefetch_hit, res_.stall_ms);
  else
    std::fprintf(f, "  residency: not measured\n");
  if (xfer_.measured)
    std::fprintf(f,
                 "  transfer: h2d %.3f GB, d2h %.3f GB, nvme read %.3f GB, nvme write %.3f GB, "
                 "peak pinned %.2f MiB\n",
                 (double)xfer_.h2d_bytes / 1e9, (double)xfer_.d2h_bytes / 1e9,
                 (double)xfer_.nvme_read_bytes / 1e9, (double)xfer_.nvme_write_bytes / 1e9,
                 (double)xfer_.peak_pinned_bytes / 1048576.0);
  else
    std::fprintf(f, "  transfer: not measured\n");
}

void Profiler::report_json(std::FILE* f) const {
  const std::vector<uint32_t> ids = by_dev_time();
  Json j(f);
  j.open(nullptr, '{');
  j.str("clock_domain", clock_domain_name(domain_));
  j.str("detail", opts_.detail);
  j.flag("subtract_floor", opts_.subtract_floor);
  j.i32("warmup_steps", opts_.warmup_steps);
  j.u64("steps_kept", count_.kept);
  j.u64("steps_discarded", count_.discarded);
  j.u64("max_depth", count_.depth);
  j.u64("nested_scopes_self_time", count_.nested);
  j.u64("ops", count_.ops);
  j.inline_open("floor");
  j.i32("n", host_floor_.n);
  j.u64("host_ns", host_floor_.ns);
  j.u64("dev_ns", dev_.enabled ? dev_.floor_ns : host_floor_.ns);
  j.inline_close();
  j.flag("device_backend", dev_.enabled);
  j.u64("device_spans", dev_.recorded);
  j.u64("device_spans_dropped", dev_.dropped);
  j.flag("device_floor_measured", dev_.floor_known);
  j.open("components", '[');
  for (uint32_t i : ids) {
    const Tally& t = tally_[i];
    j.inline_open(nullptr);
    j.str("component", names_[i]);
    j.u64("ops", t.ops);
    j.u64("dev_ns", t.dev_self);
    j.num("dev_ns_self", (double)t.dev_self - dev_floor_of(t), 1);
    j.u64("idle_ns", t.idle);
    j.u64("host_ns", t.host_self);
    j.num("host_ns_self", (double)t.host_self - host_floor_of(t), 1);
    j.inline_close();
  }
  j.close(']');
  j.flag("residency_measured", res_.measured);
  if (res_.measured) {
    j.inline_open("residency");
    j.num("vram_pct", res_.vram_pct, 4);
    j.num("ram_pct", res_.ram_pct, 4);
    j.num("nvme_pct", res_.nvme_pct, 4);
    j.u64("slots_used", res_.slots_used);
    j.u64("slots_total", res_.slots_total);
    j.u64("evictions", res_.evictions);
    j.num("prefetch_hit", res_.prefetch_hit, 4);
    j.num("stall_ms", res_.stall_ms, 4);
    j.inline_close();
  }
  j.flag("transfer_measured", xfer_.measured);
  if (xfer_.measured) {
    j.inline_open("transfer");
    j.u64("h2d_bytes", xfer_.h2d_bytes);
    j.u64("d2h_bytes", xfer_.d2h_bytes);
    j.u64("nvme_read_bytes", xfer_.nvme_read_bytes);
    j.u64("nvme_write_bytes", xfer_.nvme_write_bytes);
    j.u64("peak_pinned_bytes", xfer_.peak_pinned_bytes);
    j.inline_close();
  }
  j.close('}');
  std::fputc('\n', f);
}

void Profiler::report_csv(std::FILE* f) const {
  const std::vector<uint32_t> ids = by_dev_time();
  const uint64_t floor = dev_.enabled ? dev_.floor_ns : host_floor_.ns;
  const char* clock = clock_domain_name(domain_);
  std::fputs("component,ops,dev_ns,idle_ns,host_ns,clock_domain,detail,floor_dev_ns\n", f);
  for (uint32_t i : ids) {
    const Tally& t = tally_[i];
    std::fprintf(f, "%s,%llu,%llu,%llu,%llu,%s,%s,%llu\n", names_[i].c_str(),
                 (unsigned long long)t.ops, (unsigned long long)t.dev_self,
                 (unsigned long long)t.idle, (unsigned long long)t.host_self, clock,
                 opts_.detail.c_str(), (unsigned long long)floor);
  }
}

int Profiler::write_dir() const {
  if (opts_.dir.empty()) return 0;
  // make the directory and its parents (mkdir -p)
  std::string path;
  for (size_t i = 0; i <= opts_.dir.size(); ++i) {
    if (i == opts_.dir.size() || (opts_.dir[i] == '/' && i > 0)) {
      path = opts_.dir.substr(0, i);
      if (::mkdir(path.c_str(), 0755) != 0 && errno != EEXIST) {
        std::fprintf(stderr, "profile: no directory %s (%s)\n", path.c_str(), std::strerror(errno));
        return 0;
      }
    }
  }
  struct Out {
    const char* file;
    void (Profiler::*emit)(std::FILE*) const;
  };
  const Out outs[] = {{"profile.txt", &Profiler::report_table},
                      {"profile.json", &Profiler::report_json},
                      {"profile.csv", &Profiler::report_csv}};
  int written = 0;
  for (const Out& o : outs) {
    const std::string file = opts_.dir + "/" + o.file;
    if (std::FILE* out = std::fopen(file.c_str(), "w")) {
      (this->*o.emit)(out);
      written += std::fclose(out) == 0 ? 1 : 0;
    } else {
      std::fprintf(stderr, "profile: %s not written (%s)\n", file.c_str(), std::strerror(errno));
    }
  }
  return written;
}

void Profiler::report(std::FILE* f) const {
  if (!opts_.on) return;
  if (opts_.format == "json")
    report_json(f);
  else if (opts_.format == "csv")
    report_csv(f);
  else
    report_table(f);
}

}  // namespace knj
