// ftm_offload.cpp -- global timestamp-LRU bookkeeping of the expert slot pool.
//
// Same policy as OffloadMoeCache (python/freetoken/moe/offload_cache.py):
//   * flat id = layer * E + expert; slot_for_id[id] = slot or -1; id_of_slot[slot] = id or -1;
//     usage[slot] = step the slot was last active.
//   * ensure (decode, :560-647): step += 1; every resident routed expert is a hit and
//     stamps usage = step; the misses, in ascending expert order, each evict
//     argmin over all slots of (usage, slot) and are staged for the copy.
//   * materialize (prefill, :461-556): the same over every expert of the layer,
//     except a miss first takes the lowest free slot (id_of_slot == -1).
//   * afterwards slot_for_id is rebuilt from id_of_slot (:401-435).
// Native C++ over plain host arrays instead of per-element tensor .item() calls.
#include <stdint.h>

#include <vector>

#include "ftmoe.h"

namespace {

void resync(int32_t num_ids, int32_t cache_size, int32_t* slot_for_id, const int32_t* id_of_slot) {
  for (int32_t i = 0; i < num_ids; ++i) slot_for_id[i] = -1;
  for (int32_t s = 0; s < cache_size; ++s) {
    const int32_t id = id_of_slot[s];
    if (id >= 0 && id < num_ids) slot_for_id[id] = s;
  }
}

int32_t lru_victim(int32_t cache_size, const int64_t* usage) {
  int32_t best = 0;
  for (int32_t s = 1; s < cache_size; ++s)
    if (usage[s] < usage[best]) best = s;  // ties keep the lower slot
  return best;
}

// State arrays come from the caller: an out-of-range id or slot in them (a
// corrupt map) is skipped here, never followed, and the final resync rebuilds
// slot_for_id from id_of_slot alone.
void take_slot(int32_t victim, int32_t new_id, int64_t step, int32_t num_ids, int32_t* slot_for_id,
               int32_t* id_of_slot, int64_t* usage) {
  const int32_t old_id = id_of_slot[victim];
  if (old_id >= 0 && old_id < num_ids) slot_for_id[old_id] = -1;
  id_of_slot[victim] = new_id;
  slot_for_id[new_id] = victim;
  usage[victim] = step;
}

int check(int32_t layer_id, int32_t num_layers, int32_t num_experts, int32_t cache_size) {
  if (num_layers <= 0 || num_experts <= 0 || cache_size <= 0) return FTM_ERR_DIM;
  if (layer_id < 0 || layer_id >= num_layers) return FTM_ERR_DIM;
  return FTM_OK;
}

}  // namespace

extern "C" {

int ftm_lru_ensure(int32_t layer_id, int32_t num_layers, int32_t num_experts, int32_t cache_size,
                   const int64_t* expert_ids, int32_t n, int32_t* slot_for_id, int32_t* id_of_slot,
                   int64_t* usage, int64_t* step, int32_t* evict_slots, int32_t* src_rows,
                   int32_t* num_staged) {
  int rc = check(layer_id, num_layers, num_experts, cache_size);
  if (rc != FTM_OK) return rc;
  if (n < 0) return FTM_ERR_DIM;
  if (slot_for_id == nullptr || id_of_slot == nullptr || usage == nullptr || step == nullptr ||
      evict_slots == nullptr || src_rows == nullptr || num_staged == nullptr || (n > 0 && expert_ids == nullptr))
    return FTM_ERR_NULL;
  for (int32_t i = 0; i < n; ++i)
    if (expert_ids[i] < 0 || expert_ids[i] >= num_experts) return FTM_ERR_DIM;
  const int32_t base = layer_id * num_experts;
  // unique experts in first-appearance order (offload_cache.py:580-583)
  std::vector<uint8_t> seen_flag((size_t)num_experts, 0);
  std::vector<int32_t> seen;
  seen.reserve((size_t)n);
  for (int32_t i = 0; i < n; ++i) {
    const int32_t e = (int32_t)expert_ids[i];
    if (!seen_flag[(size_t)e]) {
      seen_flag[(size_t)e] = 1;
      seen.push_back(e);
    }
  }
  const int64_t st = *step + 1;
  *step = st;
  for (int32_t e : seen) {  // phase 1: hits
    const int32_t s = slot_for_id[base + e];
    if (s >= 0 && s < cache_size) usage[s] = st;
  }
  // phase 2: the misses, fixed before any eviction, in ascending expert id
  std::vector<int32_t> missing;
  for (int32_t e = 0; e < num_experts; ++e)
    if (seen_flag[(size_t)e] && !(slot_for_id[base + e] >= 0 && slot_for_id[base + e] < cache_size))
      missing.push_back(e);
  int32_t num = 0;
  for (int32_t e : missing) {
    const int32_t victim = lru_victim(cache_size, usage);
    take_slot(victim, base + e, st, num_layers * num_experts, slot_for_id, id_of_slot, usage);
    evict_slots[num] = victim;
    src_rows[num] = e;
    ++num;
  }
  *num_staged = num;
  resync(num_layers * num_experts, cache_size, slot_for_id, id_of_slot);
  return num;
}

int ftm_lru_materialize(int32_t layer_id, int32_t num_layers, int32_t num_experts, int32_t cache_size,
                        int32_t* slot_for_id, int32_t* id_of_slot, int64_t* usage, int64_t* step,
                        int32_t* evict_slots, int32_t* src_rows, int32_t* num_staged) {
  int rc = check(layer_id, num_layers, num_experts, cache_size);
  if (rc != FTM_OK) return rc;
  if (cache_size < num_experts) return FTM_ERR_DIM;
  if (slot_for_id == nullptr || id_of_slot == nullptr || usage == nullptr || step == nullptr ||
      evict_slots == nullptr || src_rows == nullptr || num_staged == nullptr)
    return FTM_ERR_NULL;
  const int32_t base = layer_id * num_experts;
  const int64_t st = *step + 1;
  *step = st;
  for (int32_t e = 0; e < num_experts; ++e) {
    const int32_t s = slot_for_id[base + e];
    if (s >= 0 && s < cache_size) usage[s] = st;
  }
  std::vector<int32_t> missing;
  for (int32_t e = 0; e < num_experts; ++e)
    if (!(slot_for_id[base + e] >= 0 && slot_for_id[base + e] < cache_size)) missing.push_back(e);
  int32_t num = 0;
  for (int32_t e : missing) {
    int32_t victim = -1;
    for (int32_t s = 0; s < cache_size; ++s)
      if (id_of_slot[s] == -1) {
        victim = s;
        break;
      }
    if (victim < 0) victim = lru_victim(cache_size, usage);
    take_slot(victim, base + e, st, num_layers * num_experts, slot_for_id, id_of_slot, usage);
    evict_slots[num] = victim;
    src_rows[num] = e;
    ++num;
  }
  *num_staged = num;
  resync(num_layers * num_experts, cache_size, slot_for_id, id_of_slot);
  return num;
}

}  // extern "C"
