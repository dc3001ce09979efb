// kanjoos_amd/host/knj_profiler.cpp -- the profiler of include/knj/profiler.h.
//
// Host markers are a stack of open frames; device spans are queued per stream
// and folded (sorted, nested by containment) when a report is written.  Output
// formats follow the reference's writers (/root/reference/src/profiler/
// profiler.cpp:396-517): the same CSV columns and JSON keys, so tools that read
// the reference's profile files read these.
#include "../../include/knj/profiler.h"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <filesystem>
#include <system_error>

namespace knj {
namespace {

uint64_t now_ns() {
  return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

std::string escape_json(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    if (c == '\n') {
      o += "\\n";
      continue;
    }
    o += c;
  }
  return o;
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

constexpr int kStreams = 8;
int clamp_stream(int s) { return s < 0 || s >= kStreams ? 0 : s; }

}  // namespace

const char* clock_domain_name(ClockDomain d) {
  return d == ClockDomain::Host ? "host" : d == ClockDomain::Device ? "device" : "none";
}

Profiler& Profiler::get() {
  static Profiler p;
  return p;
}

void Profiler::configure(const ProfileConfig& c) {
  cfg_ = c;
  if (cfg_.on && domain_ == ClockDomain::None) domain_ = ClockDomain::Host;
  reset();
}

void Profiler::reset() {
  rows_.clear();
  index_.clear();
  stack_.clear();
  gap_ = 0;
  std::fill(std::begin(last_end_), std::end(last_end_), 0);
  for (auto& v : pending_) v.clear();
  dev_recorded_ = dev_dropped_ = 0;
  steps_seen_ = steps_kept_ = steps_discarded_ = 0;
  nested_ops_ = max_depth_ = total_ops_ = 0;
}

size_t Profiler::row_of(const std::string& group) const {
  auto it = index_.find(group);
  if (it != index_.end()) return it->second;
  rows_.push_back(Row{group});
  index_.emplace(group, rows_.size() - 1);
  return rows_.size() - 1;
}

std::string Profiler::group_for(const char* name) const {
  std::string n = name ? name : "";
  const int keep = cfg_.detail == "class" ? 1 : cfg_.detail == "layer" ? 2 : 0;
  if (keep == 0) return n;
  size_t p = 0;
  for (int i = 0; i < keep; ++i) {
    p = n.find(':', i ? p + 1 : 0);
    if (p == std::string::npos) return n;
  }
  return n.substr(0, p);
}

void Profiler::begin(const char* name, int stream) {
  if (!cfg_.on) return;
  const uint64_t t = now_ns();
  if (stack_.empty()) {
    stream_ = clamp_stream(stream);
    const uint64_t prev = last_end_[stream_];
    gap_ = prev && t > prev ? t - prev : 0;
  } else {
    ++nested_ops_;
  }
  stack_.push_back(Frame{group_for(name), t, 0});
  max_depth_ = std::max<uint64_t>(max_depth_, stack_.size());
}

void Profiler::end() {
  if (!cfg_.on || stack_.empty()) return;
  const uint64_t t = now_ns();
  const Frame f = stack_.back();
  stack_.pop_back();
  const uint64_t span = t - f.t0;
  const uint64_t self = span > f.child_ns ? span - f.child_ns : 0;
  const bool outer = stack_.empty();
  if (outer)
    last_end_[stream_] = t;
  else
    stack_.back().child_ns += span;
  if (steps_seen_ < (uint64_t)cfg_.warmup_steps) return;
  Row& r = rows_[row_of(f.group)];
  ++r.ops;
  r.host_ns += self;
  if (!device_backend_) {  // with a device backend, dev belongs to device spans
    r.dev_ns += self;
    if (outer) r.idle_ns += gap_;
  }
  ++total_ops_;
}

void Profiler::step_done() {
  if (!cfg_.on) return;
  if (steps_seen_ < (uint64_t)cfg_.warmup_steps)
    ++steps_discarded_;
  else
    ++steps_kept_;
  ++steps_seen_;
}

void Profiler::device_span(const char* name, uint64_t start_ns, uint64_t end_ns, int stream) {
  if (!cfg_.on || !device_backend_) return;
  const size_t row = row_of(group_for(name));
  ++rows_[row].dev_spans;
  pending_[clamp_stream(stream)].push_back(Span{row, start_ns, std::max(start_ns, end_ns)});
  ++dev_recorded_;
}

// Folds queued device spans into the rows.  Per stream, spans are taken in
// start order (the longer first on a tie, so a parent precedes a child that
// starts with it); a span that starts before the innermost open span ends is
// nested in it and its time leaves the parent's self time.  A gap before an
// outermost span is that span's idle.
void Profiler::fold() const {
  struct Open {
    size_t row;
    uint64_t start, end, child;
  };
  for (auto& q : pending_) {
    if (q.empty()) continue;
    std::sort(q.begin(), q.end(), [](const Span& a, const Span& b) {
      return a.start != b.start ? a.start < b.start : a.end > b.end;
    });
    std::vector<Open> open;
    uint64_t prev_end = 0;
    bool any = false;
    auto close = [&]() {
      const Open& o = open.back();
      const uint64_t dur = o.end - o.start;
      rows_[o.row].dev_ns += dur > o.child ? dur - o.child : 0;
      open.pop_back();
    };
    for (const Span& s : q) {
      while (!open.empty() && s.start >= open.back().end) close();
      if (open.empty()) {
        if (any && s.start > prev_end) rows_[s.row].idle_ns += s.start - prev_end;
      } else {
        open.back().child += std::min(s.end, open.back().end) - s.start;
      }
      open.push_back(Open{s.row, s.start, s.end, 0});
      prev_end = any ? std::max(prev_end, s.end) : s.end;
      any = true;
    }
    while (!open.empty()) close();
    q.clear();
  }
}

void Profiler::measure_floor() {
  floor_n_ = std::max(0, cfg_.floor_ops);
  floor_host_ns_ = floor_dev_ns_ = 0;
  if (floor_n_ == 0) return;
  // the same begin/end path, on a row of its own that is removed afterwards
  const ProfileConfig keep = cfg_;
  const uint64_t keep_seen = steps_seen_, keep_ops = total_ops_, keep_nested = nested_ops_;
  const uint64_t keep_end = last_end_[kStreams - 1];
  const size_t keep_rows = rows_.size();
  cfg_.on = true;
  cfg_.detail = "kernel";
  cfg_.warmup_steps = 0;
  steps_seen_ = 0;
  for (int i = 0; i < 32; ++i) {  // warm the row and the clock
    begin("__floor", kStreams - 1);
    end();
  }
  const uint64_t t0 = now_ns();
  for (int i = 0; i < floor_n_; ++i) {
    begin("__floor", kStreams - 1);
    end();
  }
  const uint64_t t1 = now_ns();
  if (rows_.size() > keep_rows) {
    index_.erase("__floor");
    rows_.resize(keep_rows);
  }
  cfg_ = keep;
  steps_seen_ = keep_seen;
  total_ops_ = keep_ops;
  nested_ops_ = keep_nested;
  last_end_[kStreams - 1] = keep_end;
  floor_host_ns_ = (t1 - t0) / (uint64_t)floor_n_;
  floor_dev_ns_ = floor_host_ns_;  // host domain: one clock, one floor
}

std::vector<const Profiler::Row*> Profiler::ordered() const {
  fold();
  std::vector<const Row*> v;
  for (const Row& r : rows_) v.push_back(&r);
  std::sort(v.begin(), v.end(), [](const Row* a, const Row* b) {
    return a->dev_ns != b->dev_ns ? a->dev_ns > b->dev_ns : a->group < b->group;
  });
  return v;
}

// Floors are subtracted per measurement and never beyond what a row holds.
// Device rows use the device floor only once one was measured; a device-only
// row's measurements are its spans.
double Profiler::dev_floor_for(const Row& r) const {
  if (!cfg_.subtract_floor) return 0.0;
  uint64_t per = 0, n = 0;
  if (device_backend_) {
    if (!dev_floor_measured_) return 0.0;
    per = dev_floor_ns_;
    n = r.ops ? r.ops : r.dev_spans;
  } else {
    per = floor_dev_ns_;
    n = r.ops;
  }
  return std::min((double)per * (double)n, (double)r.dev_ns);
}

double Profiler::host_floor_for(const Row& r) const {
  if (!cfg_.subtract_floor) return 0.0;
  return std::min((double)floor_host_ns_ * (double)r.ops, (double)r.host_ns);
}

void Profiler::print_header(std::FILE* f, const std::string& version, const std::string& device_line,
                            const std::string& budgets_line) const {
  std::fprintf(f, "\n  kanjoos-amd %s   device %s\n", version.c_str(), device_line.c_str());
  if (!budgets_line.empty()) std::fprintf(f, "    %s\n", budgets_line.c_str());
  std::fprintf(f,
               "    clock %s; rows are self time (max depth %llu); steps kept %llu, discarded "
               "%llu (warmup %d); %llu host op(s); peak rss %.0f MiB\n",
               clock_domain_name(domain_), (unsigned long long)max_depth_,
               (unsigned long long)steps_kept_, (unsigned long long)steps_discarded_,
               cfg_.warmup_steps, (unsigned long long)total_ops_, peak_rss_mib());
  std::fprintf(f, "    profiling measures the run; it does not change what the step computes\n");
}

void Profiler::report_table(std::FILE* f) const {
  if (!cfg_.on) {
    std::fprintf(f, "\nprofile: off\n");
    return;
  }
  const auto v = ordered();
  double tdev = 0, tidle = 0, thost = 0;
  for (const Row* r : v) {
    tdev += (double)r->dev_ns - dev_floor_for(*r);
    tidle += (double)r->idle_ns;
    thost += (double)r->host_ns - host_floor_for(*r);
  }
  int w = 20;
  for (const Row* r : v) w = std::max(w, (int)r->group.size());
  std::fprintf(f, "\n  %-*s %7s %8s %7s %12s %12s %12s\n", w, "component", "ops", "spans", "%dev",
               "dev us", "idle us", "host us");
  for (const Row* r : v) {
    const double dev = (double)r->dev_ns - dev_floor_for(*r);
    std::fprintf(f, "  %-*s %7llu %8llu %6.1f%% %12.2f %12.2f %12.2f\n", w, r->group.c_str(),
                 (unsigned long long)r->ops, (unsigned long long)r->dev_spans,
                 tdev > 0 ? 100.0 * dev / tdev : 0.0, dev / 1e3, (double)r->idle_ns / 1e3,
                 ((double)r->host_ns - host_floor_for(*r)) / 1e3);
  }
  std::fprintf(f, "  total: dev %.2f us, idle %.2f us, host %.2f us\n", tdev / 1e3, tidle / 1e3,
               thost / 1e3);
  if (floor_n_ > 0)
    std::fprintf(f, "  host floor: %.3f us per marker pair (%d timed)%s\n",
                 (double)floor_host_ns_ / 1e3, floor_n_,
                 cfg_.subtract_floor ? ", subtracted" : ", not subtracted (no-subtract)");
  else
    std::fprintf(f, "  host floor: not measured\n");
  std::fprintf(f, "  clock domain: %s%s\n", clock_domain_name(domain_),
               domain_ == ClockDomain::Host ? " (dev and host are the same host interval)" : "");
  if (device_backend_) {
    std::fprintf(f, "  device spans: %llu recorded, %llu dropped%s\n",
                 (unsigned long long)dev_recorded_, (unsigned long long)dev_dropped_,
                 dev_dropped_ ? " -- the dev total is short by the dropped spans" : "");
    if (dev_floor_measured_)
      std::fprintf(f, "  device floor: %.3f us per span (%d empty kernels)%s\n",
                   (double)dev_floor_ns_ / 1e3, dev_floor_n_,
                   cfg_.subtract_floor ? ", subtracted" : ", not subtracted (no-subtract)");
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
  const auto v = ordered();
  std::fprintf(f, "{\n  \"clock_domain\": \"%s\",\n  \"detail\": \"%s\",\n",
               clock_domain_name(domain_), escape_json(cfg_.detail).c_str());
  std::fprintf(f, "  \"subtract_floor\": %s,\n  \"warmup_steps\": %d,\n",
               cfg_.subtract_floor ? "true" : "false", cfg_.warmup_steps);
  std::fprintf(f, "  \"steps_kept\": %llu,\n  \"steps_discarded\": %llu,\n",
               (unsigned long long)steps_kept_, (unsigned long long)steps_discarded_);
  std::fprintf(f, "  \"max_depth\": %llu,\n  \"nested_scopes_self_time\": %llu,\n  \"ops\": %llu,\n",
               (unsigned long long)max_depth_, (unsigned long long)nested_ops_,
               (unsigned long long)total_ops_);
  std::fprintf(f, "  \"floor\": {\"n\": %d, \"host_ns\": %llu, \"dev_ns\": %llu},\n", floor_n_,
               (unsigned long long)floor_host_ns_,
               (unsigned long long)(device_backend_ ? dev_floor_ns_ : floor_dev_ns_));
  std::fprintf(f, "  \"device_backend\": %s,\n  \"device_spans\": %llu,\n",
               device_backend_ ? "true" : "false", (unsigned long long)dev_recorded_);
  std::fprintf(f, "  \"device_spans_dropped\": %llu,\n  \"device_floor_measured\": %s,\n",
               (unsigned long long)dev_dropped_, dev_floor_measured_ ? "true" : "false");
  std::fprintf(f, "  \"components\": [\n");
  for (size_t i = 0; i < v.size(); ++i) {
    const Row& r = *v[i];
    std::fprintf(f,
                 "    {\"component\": \"%s\", \"ops\": %llu, \"dev_ns\": %llu, \"dev_ns_self\": "
                 "%.1f, \"idle_ns\": %llu, \"host_ns\": %llu, \"host_ns_self\": %.1f}%s\n",
                 escape_json(r.group).c_str(), (unsigned long long)r.ops,
                 (unsigned long long)r.dev_ns, (double)r.dev_ns - dev_floor_for(r),
                 (unsigned long long)r.idle_ns, (unsigned long long)r.host_ns,
                 (double)r.host_ns - host_floor_for(r), i + 1 < v.size() ? "," : "");
  }
  std::fprintf(f, "  ],\n  \"residency_measured\": %s,\n", res_.measured ? "true" : "false");
  if (res_.measured)
    std::fprintf(f,
                 "  \"residency\": {\"vram_pct\": %.4f, \"ram_pct\": %.4f, \"nvme_pct\": %.4f, "
                 "\"slots_used\": %llu, \"slots_total\": %llu, \"evictions\": %llu, "
                 "\"prefetch_hit\": %.4f, \"stall_ms\": %.4f},\n",
                 res_.vram_pct, res_.ram_pct, res_.nvme_pct, (unsigned long long)res_.slots_used,
                 (unsigned long long)res_.slots_total, (unsigned long long)res_.evictions,
                 res_.prefetch_hit, res_.stall_ms);
  std::fprintf(f, "  \"transfer_measured\": %s", xfer_.measured ? "true" : "false");
  if (xfer_.measured)
    std::fprintf(f,
                 ",\n  \"transfer\": {\"h2d_bytes\": %llu, \"d2h_bytes\": %llu, "
                 "\"nvme_read_bytes\": %llu, \"nvme_write_bytes\": %llu, \"peak_pinned_bytes\": "
                 "%llu}",
                 (unsigned long long)xfer_.h2d_bytes, (unsigned long long)xfer_.d2h_bytes,
                 (unsigned long long)xfer_.nvme_read_bytes,
                 (unsigned long long)xfer_.nvme_write_bytes,
                 (unsigned long long)xfer_.peak_pinned_bytes);
  std::fprintf(f, "\n}\n");
}

void Profiler::report_csv(std::FILE* f) const {
  const auto v = ordered();
  std::fprintf(f, "component,ops,dev_ns,idle_ns,host_ns,clock_domain,detail,floor_dev_ns\n");
  const uint64_t floor = device_backend_ ? dev_floor_ns_ : floor_dev_ns_;
  for (const Row* r : v)
    std::fprintf(f, "%s,%llu,%llu,%llu,%llu,%s,%s,%llu\n", r->group.c_str(),
                 (unsigned long long)r->ops, (unsigned long long)r->dev_ns,
                 (unsigned long long)r->idle_ns, (unsigned long long)r->host_ns,
                 clock_domain_name(domain_), cfg_.detail.c_str(), (unsigned long long)floor);
}

int Profiler::write_dir() const {
  if (cfg_.dir.empty()) return 0;
  std::error_code ec;
  std::filesystem::create_directories(cfg_.dir, ec);
  if (ec && !std::filesystem::is_directory(cfg_.dir)) {
    std::fprintf(stderr, "profile-dir: cannot create %s: %s\n", cfg_.dir.c_str(),
                 ec.message().c_str());
    return 0;
  }
  int n = 0;
  const char* names[3] = {"profile.txt", "profile.json", "profile.csv"};
  for (int i = 0; i < 3; ++i) {
    const std::string path = cfg_.dir + "/" + names[i];
    std::FILE* out = std::fopen(path.c_str(), "w");
    if (!out) {
      std::fprintf(stderr, "profile-dir: cannot write %s\n", path.c_str());
      continue;
    }
    if (i == 0)
      report_table(out);
    else if (i == 1)
      report_json(out);
    else
      report_csv(out);
    std::fclose(out);
    ++n;
  }
  return n;
}

void Profiler::report(std::FILE* f) const {
  if (!cfg_.on) return;
  if (cfg_.format == "json")
    report_json(f);
  else if (cfg_.format == "csv")
    report_csv(f);
  else
    report_table(f);
}

}  // namespace knj
