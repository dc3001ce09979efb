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
  const ProfileConfig& config() const { return opts_; }
  bool on() const { return opts_.on; }

  // Marker pair.  `name` is "class", "class:layer" or "class:layer:kernel";
  // detail "class" keeps the part before the first ':', "layer" the part
  // before the second, "kernel" all of it.
  void begin(const char* name, int stream = 0);
  void end();
  void step_done();

  void set_domain(ClockDomain d) { domain_ = d; }
  ClockDomain domain() const { return domain_; }

  void enable_device_backend();
  bool device_backend() const { return dev_.enabled; }
  // One device interval, as offsets (ns) from the stream's epoch event.
  void device_span(const char* name, uint64_t start_ns, uint64_t end_ns, int stream = 0);
  void set_device_floor(uint64_t ns, int n);
  bool device_floor_measured() const { return dev_.floor_known; }
  void set_device_dropped(uint64_t spans) { dev_.dropped = spans; }
  uint64_t device_spans() const { return dev_.recorded; }
  uint64_t device_dropped() const { return dev_.dropped; }

  void note_residency(const ResidencyStats& r) { res_ = r; }
  void note_transfer(const TransferStats& t) { xfer_ = t; }

  void measure_floor();
  uint64_t floor_host_ns() const { return host_floor_.ns; }
  uint64_t floor_dev_ns() const { return host_floor_.ns; }  // host domain: one clock
  int floor_n() const { return host_floor_.n; }

  uint64_t steps_kept() const { return count_.kept; }
  uint64_t steps_discarded() const { return count_.discarded; }
  uint64_t nested_ops() const { return count_.nested; }
  uint64_t max_depth() const { return count_.depth; }
  uint64_t op_count() const { return count_.ops; }

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

  // Everything measured is an interval on a lane: a host-marker lane (the
  // stream named by the outermost open marker) or a device stream.  Closed
  // intervals are logged and turned into per-component tallies by one sweep
  // (settle()), the same for both sources: sorted by start, a containment
  // stack gives each interval's children (self time) and each outermost
  // interval's gap to the previous one on its lane (idle).
  enum class Source : uint8_t { Host = 0, Device = 1 };
  static constexpr int kLanes = 8;
  struct Interval {
    uint32_t comp;
    uint8_t lane;
    Source src;
    bool counted;  // false: closed during warmup (still shapes nesting and idle)
    uint64_t t0, t1, seq;
  };
  struct Tally {
    uint64_t ops = 0, spans = 0;              // host intervals, device intervals
    uint64_t host_self = 0, dev_self = 0, idle = 0;
  };
  struct OpenMarker {
    uint32_t comp;
    uint64_t t0, seq;
  };
  struct LaneEdge {
    bool any = false;
    uint64_t last_end = 0;  // end of the last outermost interval swept
  };
  struct DeviceInfo {
    bool enabled = false, floor_known = false;
    uint64_t floor_ns = 0;
    int floor_n = 0;
    uint64_t recorded = 0, dropped = 0;
  };
  struct HostFloor {
    int n = 0;
    uint64_t ns = 0;
  };
  struct Counters {
    uint64_t steps = 0, kept = 0, discarded = 0;
    uint64_t nested = 0, depth = 0, ops = 0, seq = 0;
  };

  uint32_t component(const char* name) const;  // interned at the configured detail
  void settle() const;                         // sweeps the logged intervals
  std::vector<uint32_t> by_dev_time() const;
  double dev_floor_of(const Tally& t) const;
  double host_floor_of(const Tally& t) const;

  ProfileConfig opts_;
  ClockDomain domain_ = ClockDomain::None;
  mutable std::vector<std::string> names_;
  mutable std::unordered_map<std::string, uint32_t> ids_;
  mutable std::vector<Tally> tally_;
  mutable std::vector<Interval> log_;
  mutable LaneEdge edge_[2][kLanes];
  std::vector<OpenMarker> open_;
  uint8_t open_lane_ = 0;
  Counters count_;
  DeviceInfo dev_;
  HostFloor host_floor_;
  ResidencyStats res_;
  TransferStats xfer_;
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
