// kanjoos_amd/host/knj_residency.cpp -- the all-resident ResidencyManager of
// include/knj/residency.h.
#include "../../include/knj/residency.h"

namespace knj {

const char* to_string(Residency r) {
  static const char* names[] = {"ABSENT",        "NVME_RESIDENT", "LOADING_NVME", "RAM_RESIDENT",
                                "LOADING_RAM",   "VRAM_RESIDENT", "PREFETCHED",   "EVICTING_VRAM",
                                "EVICTING_RAM",  "PINNED",        "INVALID"};
  const unsigned i = (unsigned)r;
  return i < sizeof(names) / sizeof(names[0]) ? names[i] : "?";
}

ResidencyManager::ResidencyManager(uint32_t n_layer, uint32_t n_expert, uint32_t n_ctx,
                                   uint32_t kv_page_tokens)
    : n_layer_(n_layer),
      n_expert_(n_expert),
      n_pages_(kv_page_tokens ? (n_ctx + kv_page_tokens - 1) / kv_page_tokens : 0) {}

// Nothing to move: the object is already in VRAM.  An unknown id is a caller
// error the reference would also refuse to serve; it counts as a miss.
void ResidencyManager::request(ExpertId id, KVTier) {
  if (!known(id)) ++misses_;
}
void ResidencyManager::prefetch(ExpertId id, KVTier, PrefetchPriority) {
  if (!known(id)) ++misses_;
}
void ResidencyManager::promote(ExpertId) {}
void ResidencyManager::demote(ExpertId id) {
  if (known(id)) ++refused_;  // pinned: eviction is refused, not ignored
}
void ResidencyManager::tick() { ++tick_; }
void ResidencyManager::pin(ExpertId) {}
void ResidencyManager::unpin(ExpertId) {}

void ResidencyManager::request_kv(KvPageId id, KVTier) {
  if (!known_kv(id)) ++misses_;
}
void ResidencyManager::prefetch_kv(KvPageId id, KVTier, PrefetchPriority) {
  if (!known_kv(id)) ++misses_;
}
void ResidencyManager::promote_kv(KvPageId) {}
void ResidencyManager::demote_kv(KvPageId id) {
  if (known_kv(id)) ++refused_;
}

bool ResidencyManager::demand(ExpertId id, KVTier) {
  ++demands_;
  if (known(id)) return true;
  ++misses_;
  return false;
}

bool ResidencyManager::demand_kv(KvPageId id, KVTier) {
  ++demands_;
  if (known_kv(id)) return true;
  ++misses_;
  return false;
}

void ResidencyManager::reset() {
  layer_ = 0;
  tick_ = misses_ = refused_ = demands_ = 0;
}

ResidencyStats ResidencyManager::stats() const {
  ResidencyStats r;
  r.measured = true;
  r.vram_pct = 100.0;
  r.slots_used = r.slots_total = (uint64_t)n_layer_ * n_expert_;
  r.evictions = 0;
  r.prefetch_hit = demands_ ? (double)(demands_ - misses_) / (double)demands_ : 1.0;
  r.stall_ms = 0.0;
  return r;
}

}  // namespace knj
