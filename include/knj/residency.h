// include/knj/residency.h -- the residency contract as a pass-through for a
// model that lives in HBM whole.
//
// The reference's ResidencyManager (/root/reference/src/residency/
// residency.h:254-369) moves experts and KV pages between NVMe, host RAM and
// VRAM slots, one tick per layer.  On a 288 GB MI355X the whole Qwen3-30B-A3B
// image (about 17 GB at Q4_K) and its KV cache are resident from load to exit,
// so every object starts and stays PINNED in VRAM.  This class keeps the
// reference's API and counters so callers written against it run unchanged:
// locate() answers PINNED, ready()/demand() answer true and count a hit,
// request()/prefetch()/promote() have nothing to move, demote() is refused
// (a pinned object is never an eviction candidate, as in the reference), and
// stats() reports the residency row the profiler prints (100% VRAM, every slot
// used, no evictions, no stalls).
#pragma once

#include <cstdint>
#include <vector>

#include "profiler.h"

namespace knj {

struct ExpertId {
  uint32_t layer = 0;
  uint32_t index = 0;
  uint64_t key() const { return ((uint64_t)layer << 32) | index; }
  bool operator==(const ExpertId& o) const { return key() == o.key(); }
};

struct KvPageId {
  uint32_t layer = 0;
  uint32_t page = 0;
  uint64_t key() const { return ((uint64_t)layer << 32) | page; }
  bool operator==(const KvPageId& o) const { return key() == o.key(); }
};

// The reference's eleven states; this pass-through uses ABSENT and PINNED.
enum class Residency : uint8_t {
  ABSENT = 0,
  NVME_RESIDENT,
  LOADING_NVME,
  RAM_RESIDENT,
  LOADING_RAM,
  VRAM_RESIDENT,
  PREFETCHED,
  EVICTING_VRAM,
  EVICTING_RAM,
  PINNED,
  INVALID
};
const char* to_string(Residency r);

enum class KVTier : uint8_t { NVME = 0, RAM = 1, VRAM = 2 };
enum class PrefetchPriority : uint8_t { BACKGROUND = 0, NORMAL = 1, URGENT = 2 };

class ResidencyManager {
 public:
  // Every expert of every layer and every KV page of `kv_page_tokens` tokens
  // up to n_ctx is registered resident.
  ResidencyManager(uint32_t n_layer, uint32_t n_expert, uint32_t n_ctx, uint32_t kv_page_tokens);

  size_t n_experts() const { return (size_t)n_layer_ * n_expert_; }
  size_t n_kv_pages() const { return (size_t)n_layer_ * n_pages_; }
  bool known(ExpertId id) const { return id.layer < n_layer_ && id.index < n_expert_; }
  bool known_kv(KvPageId id) const { return id.layer < n_layer_ && id.page < n_pages_; }

  Residency locate(ExpertId id) const { return known(id) ? Residency::PINNED : Residency::ABSENT; }
  void request(ExpertId id, KVTier tier);
  void prefetch(ExpertId id, KVTier tier, PrefetchPriority prio);
  void promote(ExpertId id);
  void demote(ExpertId id);
  void tick();
  bool ready(ExpertId id) const { return known(id); }
  void pin(ExpertId id);
  void unpin(ExpertId id);

  Residency locate_kv(KvPageId id) const {
    return known_kv(id) ? Residency::PINNED : Residency::ABSENT;
  }
  void request_kv(KvPageId id, KVTier tier);
  void prefetch_kv(KvPageId id, KVTier tier, PrefetchPriority prio);
  void promote_kv(KvPageId id);
  void demote_kv(KvPageId id);
  bool ready_kv(KvPageId id) const { return known_kv(id); }

  void begin_layer(uint32_t layer) { layer_ = layer; }
  uint32_t layer() const { return layer_; }
  uint64_t tick_index() const { return tick_; }

  // Demand for a routed contribution: true when usable now (always, for a
  // known object); an unknown id counts a miss and returns false.
  bool demand(ExpertId id, KVTier tier);
  bool demand_or_fallback(ExpertId id) { return demand(id, KVTier::VRAM); }
  bool demand_kv(KvPageId id, KVTier tier);
  bool demand_kv_or_fallback(KvPageId id) { return demand_kv(id, KVTier::VRAM); }

  // Nothing is ever evictable.
  const std::vector<ExpertId>& eviction_candidates() const { return no_experts_; }
  const std::vector<KvPageId>& kv_eviction_candidates() const { return no_pages_; }

  void reset();

  uint64_t transitions() const { return 0; }
  uint64_t deadline_misses() const { return misses_; }
  uint64_t preempted_prefetches() const { return 0; }
  uint64_t refused_demotions() const { return refused_; }
  uint64_t tick_calls() const { return tick_; }
  uint64_t entry_visits() const { return 0; }
  uint64_t demands() const { return demands_; }
  static constexpr uint64_t blocking_transfer_calls() { return 0; }

  // The row the profiler prints for this run.
  ResidencyStats stats() const;

  // What a kernel may ask: ready() only.
  class KernelView {
   public:
    explicit KernelView(const ResidencyManager* m) : m_(m) {}
    bool ready(ExpertId id) const { return m_->ready(id); }
    bool ready_kv(KvPageId id) const { return m_->ready_kv(id); }

   private:
    const ResidencyManager* m_;
  };
  KernelView kernel_view() const { return KernelView(this); }

 private:
  uint32_t n_layer_, n_expert_, n_pages_;
  uint32_t layer_ = 0;
  uint64_t tick_ = 0, misses_ = 0, refused_ = 0, demands_ = 0;
  std::vector<ExpertId> no_experts_;
  std::vector<KvPageId> no_pages_;
};

}  // namespace knj
