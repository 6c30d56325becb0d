// Expert placement of the host-CPU hybrid (placement.h), and its C ABI for host-side use and tests.
#include "placement.h"

#include <math.h>

#include <algorithm>
#include <new>

#include "../../include/moert.h"

namespace moert {
int set_error(int code, const char* fmt, ...);

Freq::Freq(int keys, int layers)
    : lv((size_t)keys, -INFINITY), step((size_t)keys, 0), per(kHalfLife * (double)layers) {}

// Freq::touch (cache.rs:48-53): the value decayed from its last update to step s, plus one, kept as log2
void Freq::touch(int key, uint64_t s) {
  const double l = lv[key];
  const double v = l > -INFINITY ? exp2(l - (double)(s - step[key]) / per) : 0.0;
  lv[key] = log2(v + 1.0);
  step[key] = s;
}

void Freq::clear() {
  std::fill(lv.begin(), lv.end(), -INFINITY);
  std::fill(step.begin(), step.end(), 0);
}

Placement::Placement(int layers, int experts, int top_k, int slots, int backlog)
    : L_(layers), E_(experts), K_(top_k), backlog_(backlog), slot_((size_t)slots), key_slot_((size_t)layers * experts, -1),
      version_((size_t)layers * experts, 0), table_((size_t)layers * experts, -1), freq_(layers * experts, layers) {}

void Placement::start() { publish(); }

void Placement::publish() {
  std::fill(table_.begin(), table_.end(), -1);
  for (size_t i = 0; i < slot_.size(); i++)
    if (slot_[i].kind == RESIDENT) table_[slot_[i].key] = (int)i;
}

int Placement::resident() const {
  int n = 0;
  for (const Slot& s : slot_) n += s.kind == RESIDENT;
  return n;
}

// copies of this token not landed yet (the barrier mode counts every one, held or queued)
int Placement::pending() const {
  int n = 0;
  for (const Slot& s : slot_) n += s.kind == LOADING || s.kind == HELD;
  return n;
}

// the copies held for victims of `layer` are queued now, in the order they were admitted
void Placement::release_held(int layer) {
  std::vector<int> keep;
  for (int s : held_order_) {
    if (slot_[s].kind == HELD && slot_[s].after == layer) {
      slot_[s].kind = LOADING;
      copies_.push_back({s, slot_[s].key});
    } else {
      keep.push_back(s);
    }
  }
  held_order_.swap(keep);
}

void Placement::serve_layer(int l, const int* ids, int m, std::vector<int>* union_keys, std::vector<int>* union_n,
                            std::vector<char>* gpu) {
  cur_layer_ = l;
  if (l > 0) release_held(l - 1);
  std::vector<int> keys, n_e;
  for (int p = 0; p < m; p++)
    for (int j = 0; j < K_; j++) {
      const int key = l * E_ + ids[(size_t)p * K_ + j];
      const auto it = std::find(keys.begin(), keys.end(), key);
      if (it == keys.end()) {
        keys.push_back(key);
        n_e.push_back(1);
      } else {
        n_e[it - keys.begin()]++;
      }
    }
  // all of this layer's requests are recorded in the frequency table with one timestamp (step_), ahead of the
  // placement decisions below; afterwards the timestamp advances by the m positions of the block
  for (size_t i = 0; i < keys.size(); i++)
    for (int r = 0; r < n_e[i]; r++) freq_.touch(keys[i], step_);
  step_ += (uint64_t)m;
  misses_.clear();
  if (gpu) gpu->assign(keys.size(), 0);
  for (size_t i = 0; i < keys.size(); i++) {
    const int k = keys[i];
    stats_.needed += (uint64_t)n_e[i];
    if (table_[k] >= 0) {
      stats_.hits += (uint64_t)n_e[i];
      const int s = key_slot_[k];
      if (s >= 0 && slot_[s].kind == RESIDENT && slot_[s].key == k) version_[k]++;
      if (gpu) (*gpu)[i] = 1;
    } else {
      stats_.cpu += (uint64_t)n_e[i];
      if (key_slot_[k] < 0) misses_.push_back(k);
    }
  }
  layer_keys_ = keys;
  if (union_keys) *union_keys = keys;
  if (union_n) *union_n = n_e;
}

void Placement::admit_layer() {
  for (int cand : misses_) {
    if (slot_.empty() || pending() >= backlog_) {
      stats_.dropped++;
      continue;
    }
    int slot = -1, evicted = -1;
    for (size_t i = 0; i < slot_.size() && slot < 0; i++)
      if (slot_[i].kind == FREE) slot = (int)i;
    if (slot < 0) {
      // the weakest resident outside the layer's keys, by (score, version, key)
      int best = -1;
      double bs = 0;
      for (size_t i = 0; i < slot_.size(); i++) {
        if (slot_[i].kind != RESIDENT) continue;
        const int key = slot_[i].key;
        if (std::find(layer_keys_.begin(), layer_keys_.end(), key) != layer_keys_.end()) continue;
        const double sc = freq_.score(key);
        const int bk = best >= 0 ? slot_[best].key : -1;
        if (best < 0 || sc < bs || (sc == bs && (version_[key] < version_[bk] || (version_[key] == version_[bk] && key < bk)))) {
          best = (int)i;
          bs = sc;
        }
      }
      if (best < 0 || !(bs < freq_.score(cand))) {
        stats_.dropped++;
        continue;
      }
      evicted = slot_[best].key;
      key_slot_[evicted] = -1;
      slot = best;
    }
    // copy_after_reader: a victim of a layer that has not passed in this token keeps its data until that layer ends
    stats_.copies++;
    key_slot_[cand] = slot;
    slot_[slot].key = cand;
    if (evicted >= 0 && evicted / E_ >= cur_layer_) {
      slot_[slot].kind = HELD;
      slot_[slot].after = evicted / E_;
      held_order_.push_back(slot);
      stats_.deferred++;
    } else {
      slot_[slot].kind = LOADING;
      slot_[slot].after = -1;
      copies_.push_back({slot, cand});
    }
  }
  misses_.clear();
}

void Placement::end_token() {
  release_held(L_ - 1);
  for (Slot& s : slot_)
    if (s.kind == LOADING) {
      s.kind = RESIDENT;
      version_[s.key]++;
    }
  publish();
}

std::vector<CopyOrder> Placement::take_copies() {
  std::vector<CopyOrder> out;
  out.swap(copies_);
  return out;
}

}  // namespace moert

// ---- C ABI ----
using moert::Placement;
using moert::set_error;

struct moert_placement {
  Placement p;
  int L, E, K;
  bool started = false;
};

struct moert_freq {
  moert::Freq f;
};

extern "C" {

int moert_placement_create(int layers, int experts, int top_k, int slots, int backlog, moert_placement** out) {
  if (!out) return set_error(MOERT_E_CONFIG, "placement: null output");
  *out = nullptr;
  if (layers < 1 || experts < 1 || top_k < 1 || top_k > experts || slots < 0 || slots > layers * experts || backlog < 0)
    return set_error(MOERT_E_CONFIG, "placement: layers %d, experts %d, top_k %d, slots %d, backlog %d", layers, experts,
                     top_k, slots, backlog);
  moert_placement* p = new (std::nothrow) moert_placement{Placement(layers, experts, top_k, slots, backlog), layers,
                                                          experts, top_k};
  if (!p) return set_error(MOERT_E_CONFIG, "placement: out of memory");
  *out = p;
  return MOERT_OK;
}

int moert_placement_destroy(moert_placement* p) {
  delete p;
  return MOERT_OK;
}

int moert_placement_step(moert_placement* p, const int* ids, int m, int* gpu_requests, int* copies) {
  if (!p || !ids || m < 1) return set_error(MOERT_E_CONFIG, "placement step: null handle or ids, or m < 1");
  const size_t per_layer = (size_t)m * p->K;
  for (size_t i = 0; i < per_layer * p->L; i++)
    if (ids[i] < 0 || ids[i] >= p->E) return set_error(MOERT_E_RANGE, "placement step: expert id %d", ids[i]);
  for (int l = 0; l < p->L; l++)
    for (int q = 0; q < m; q++)
      for (int a = 0; a < p->K; a++)
        for (int b = a + 1; b < p->K; b++)
          if (ids[l * per_layer + (size_t)q * p->K + a] == ids[l * per_layer + (size_t)q * p->K + b])
            return set_error(MOERT_E_CONFIG, "placement step: a position routes expert %d twice",
                             ids[l * per_layer + (size_t)q * p->K + a]);
  if (!p->started) {
    p->p.start();
    p->started = true;
  }
  int on_gpu = 0, n_copies = 0;
  std::vector<int> keys, n_e;
  std::vector<char> gpu;
  for (int l = 0; l < p->L; l++) {
    p->p.serve_layer(l, ids + l * per_layer, m, &keys, &n_e, &gpu);
    for (size_t i = 0; i < keys.size(); i++) on_gpu += gpu[i] ? n_e[i] : 0;
    p->p.admit_layer();
    n_copies += (int)p->p.take_copies().size();
  }
  p->p.end_token();
  n_copies += (int)p->p.take_copies().size();
  if (gpu_requests) *gpu_requests = on_gpu;
  if (copies) *copies = n_copies;
  return MOERT_OK;
}

int moert_placement_counters(const moert_placement* p, moert_cache_counters* out) {
  if (!p || !out) return set_error(MOERT_E_CONFIG, "placement counters: null argument");
  const moert::PlacementStats& s = p->p.stats();
  moert_cache_counters c{};
  c.needed = s.needed;
  c.hits = s.hits;
  c.cpu = s.cpu;
  c.copies = s.copies;
  c.dropped = s.dropped;
  c.deferred = s.deferred;
  c.slots = p->p.slots();
  *out = c;
  return MOERT_OK;
}

int moert_placement_table(const moert_placement* p, int* table) {
  if (!p || !table) return set_error(MOERT_E_CONFIG, "placement table: null argument");
  const std::vector<int>& t = p->p.table();
  std::copy(t.begin(), t.end(), table);
  return MOERT_OK;
}

int moert_freq_create(int keys, int layers, moert_freq** out) {
  if (!out || keys < 1 || layers < 1) return set_error(MOERT_E_CONFIG, "freq: %d keys, %d layers", keys, layers);
  *out = new (std::nothrow) moert_freq{moert::Freq(keys, layers)};
  return *out ? MOERT_OK : set_error(MOERT_E_CONFIG, "freq: out of memory");
}

int moert_freq_destroy(moert_freq* f) {
  delete f;
  return MOERT_OK;
}

int moert_freq_touch(moert_freq* f, int key, uint64_t step) {
  if (!f || key < 0 || key >= (int)f->f.lv.size()) return set_error(MOERT_E_RANGE, "freq touch: key %d", key);
  if (step < f->f.step[key]) return set_error(MOERT_E_CONFIG, "freq touch: step %llu before the key's last update",
                                              (unsigned long long)step);
  f->f.touch(key, step);
  return MOERT_OK;
}

int moert_freq_score(const moert_freq* f, int key, double* score) {
  if (!f || !score || key < 0 || key >= (int)f->f.lv.size()) return set_error(MOERT_E_RANGE, "freq score: key %d", key);
  *score = f->f.score(key);
  return MOERT_OK;
}

int moert_freq_clear(moert_freq* f) {
  if (!f) return set_error(MOERT_E_CONFIG, "freq clear: null handle");
  f->f.clear();
  return MOERT_OK;
}

}  // extern "C"
