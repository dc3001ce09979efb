// include/knj/profiler.h -- op-level profiling of the decode step, host markers
// plus a device-event backend.
//
// Same interface as the reference's profiler (/root/reference/src/profiler/
// profiler.h:44-253): ProfileConfig, ClockDomain, Profiler::get(),
// begin/end markers (KNJ_PROFILE_OP), step_done() with warmup discard,
// enable_device_backend() / device_span() / set_device_floor() /
// set_device_dropped(), measure_floor(), note_residency()/note_transfer(), and
// the table / JSON / CSV writers with the same CSV columns and JSON keys.
//
// Definitions the numbers follow:
//  * Rows are SELF time.  A host marker opened inside another subtracts its
//    interval from its parent; a device span contained in another span of the
//    same stream does the same.  The rows therefore partition the measured time.
//  * `idle` is a gap between OUTERMOST intervals of one stream, charged to the
//    row of the interval that follows it.  A gap inside an open interval is not
//    idle.  Streams have separate gaps.
//  * Clock domain.  Without a device backend, `dev` and `host` are the same
//    host interval (ClockDomain::Host).  With one (ClockDomain::Device), host
//    markers write `host` only and `dev`/`idle` come from device spans, which
//    are offsets from one epoch event per stream.  On this build the spans are
//    dispatch-recorded HIP events around each kernel launch
//    (knj_model_profile), so `dev` is kernel execution time and `idle` is the
//    time the stream had no kernel running.
//  * Floors.  measure_floor() times empty marker pairs (the host floor); a
//    device floor is measured separately through the event path
//    (knj_device_floor) and handed in with set_device_floor().  Subtraction is
//    per measurement, never more than the row holds, and a host floor is never
//    subtracted from device time.
//  * A span the caller could not record is reported as dropped.
//
// The profiler itself makes no HIP call: device spans are plain numbers, so
// its arithmetic is testable without a GPU.
#pragma once

#include <cstdint>
#include <cstdio>
#include <string>
#include <unordered_map>
#include <vector>

namespace knj {

struct ProfileConfig {
  bool on = false;
  std::string format = "table";  // table | json | csv
  std::string detail = "class";  // class | layer | kernel
  std::string dir;               // write profile.{txt,json,csv} here when set
  int floor_ops = 256;           // empty marker pairs timed by measure_floor()
  int warmup_steps = 8;          // steps whose ops are discarded
  bool subtract_floor = true;    // false: --profiling=no-subtract
};

enum class ClockDomain { None, Host, Device };
const char* clock_domain_name(ClockDomain d);

// Residency and transfer counters; `measured` false prints "not measured".
struct ResidencyStats {
  bool measured = false;
  double vram_pct = 0.0, ram_pct = 0.0, nvme_pct = 0.0;
  uint64_t slots_used = 0, slots_total = 0, evictions = 0;
  double prefetch_hit = 0.0, stall_ms = 0.0;
};

struct TransferStats {
  bool measured = false;
  uint64_t h2d_bytes = 0, d2h_bytes = 0, nvme_read_bytes = 0, nvme_write_bytes = 0;
  uint64_t peak_pinned_bytes = 0;
};

class Profiler {
 public:
  static Profiler& get();

  void configure(const ProfileConfig& c);
  const ProfileConfig& config() const { return cfg_; }
  bool on() const { return cfg_.on; }

  // Marker pair.  `name` is "class", "class:layer" or "class:layer:kernel";
  // detail "class" keeps the part before the first ':', "layer" the part
  // before the second, "kernel" all of it.
  void begin(const char* name, int stream = 0);
  void end();
  void step_done();

  void set_domain(ClockDomain d) { domain_ = d; }
  ClockDomain domain() const { return domain_; }

  void enable_device_backend() {
    device_backend_ = true;
    domain_ = ClockDomain::Device;
  }
  bool device_backend() const { return device_backend_; }
  // One device interval, as offsets (ns) from the stream's epoch event.
  void device_span(const char* name, uint64_t start_ns, uint64_t end_ns, int stream = 0);
  void set_device_floor(uint64_t ns, int n) {
    dev_floor_ns_ = ns;
    dev_floor_n_ = n;
    dev_floor_measured_ = true;
  }
  bool device_floor_measured() const { return dev_floor_measured_; }
  void set_device_dropped(uint64_t spans) { dev_dropped_ = spans; }
  uint64_t device_spans() const { return dev_recorded_; }
  uint64_t device_dropped() const { return dev_dropped_; }

  void note_residency(const ResidencyStats& r) { res_ = r; }
  void note_transfer(const TransferStats& t) { xfer_ = t; }

  void measure_floor();
  uint64_t floor_host_ns() const { return floor_host_ns_; }
  uint64_t floor_dev_ns() const { return floor_dev_ns_; }
  int floor_n() const { return floor_n_; }

  uint64_t steps_kept() const { return steps_kept_; }
  uint64_t steps_discarded() const { return steps_discarded_; }
  uint64_t nested_ops() const { return nested_ops_; }
  uint64_t max_depth() const { return max_depth_; }
  uint64_t op_count() const { return total_ops_; }

  void print_header(std::FILE* f, const std::string& version, const std::string& device_line,
                    const std::string& budgets_line) const;
  void report_table(std::FILE* f) const;
  void report_json(std::FILE* f) const;
  void report_csv(std::FILE* f) const;
  int write_dir() const;
  void report(std::FILE* f) const;

  void reset();

 private:
  Profiler() = default;

  struct Row {
    std::string group;
    uint64_t ops = 0, dev_ns = 0, idle_ns = 0, host_ns = 0;
    uint64_t dev_spans = 0;  // device measurements in the row
  };
  struct Frame {
    std::string group;
    uint64_t t0, child_ns;
  };
  struct Span {
    size_t row;
    uint64_t start, end;
  };

  size_t row_of(const std::string& group) const;  // creates the row
  std::string group_for(const char* name) const;
  void fold() const;
  std::vector<const Row*> ordered() const;
  double dev_floor_for(const Row& r) const;   // ns to subtract from dev
  double host_floor_for(const Row& r) const;  // ns to subtract from host

  ProfileConfig cfg_;
  ClockDomain domain_ = ClockDomain::None;
  mutable std::vector<Row> rows_;
  mutable std::unordered_map<std::string, size_t> index_;
  std::vector<Frame> stack_;
  int stream_ = 0;
  uint64_t gap_ = 0;
  uint64_t last_end_[8] = {};
  uint64_t steps_seen_ = 0, steps_kept_ = 0, steps_discarded_ = 0;
  uint64_t nested_ops_ = 0, max_depth_ = 0, total_ops_ = 0;
  uint64_t floor_host_ns_ = 0, floor_dev_ns_ = 0;
  int floor_n_ = 0;
  ResidencyStats res_;
  TransferStats xfer_;
  bool device_backend_ = false, dev_floor_measured_ = false;
  uint64_t dev_floor_ns_ = 0;
  int dev_floor_n_ = 0;
  uint64_t dev_recorded_ = 0, dev_dropped_ = 0;
  mutable std::vector<Span> pending_[8];
};

// RAII marker.
class ProfileOp {
 public:
  explicit ProfileOp(const char* name, int stream = 0) { Profiler::get().begin(name, stream); }
  ~ProfileOp() { Profiler::get().end(); }
  ProfileOp(const ProfileOp&) = delete;
  ProfileOp& operator=(const ProfileOp&) = delete;
};

}  // namespace knj

#define KNJ_PROFILE_JOIN_(a, b) a##b
#define KNJ_PROFILE_JOIN(a, b) KNJ_PROFILE_JOIN_(a, b)
#define KNJ_PROFILE_OP(name) ::knj::ProfileOp KNJ_PROFILE_JOIN(knj_prof_, __COUNTER__)(name)
#define KNJ_PROFILE_OP_STREAM(name, stream) \
  ::knj::ProfileOp KNJ_PROFILE_JOIN(knj_prof_, __COUNTER__)(name, stream)
