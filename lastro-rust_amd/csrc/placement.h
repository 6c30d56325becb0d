// Expert placement of the host-CPU hybrid (host only): which experts of a layer step the GPU computes from the HBM
// pool and which the host computes, and which missed experts are admitted into the pool. Replaces the service line
// of the reference's D1 engine in its deterministic mode (rust/moe-rt/src/motor/line.rs: serve_layer 512-583, victim
// 605-648, copy_after_reader 653-674, end_token 678-716, with AdmitMode::TokenBarrier and the LfuCpu policy) and its
// decayed frequency (Freq, rust/moe-rt/src/cache.rs:60-87).
//
// A token (a step of m positions) reads the table published when it starts: the experts resident then are computed
// on the GPU, every other request on the host. After a layer's host work, each missed key that has no slot yet is
// admitted when the backlog (copies queued in this token) is below its bound and a slot is free or the weakest
// resident outside the layer's own keys (lowest (score, version, key)) scores below it. A copy into the slot of a
// victim whose layer has not yet run in this token is held until that layer has passed. At the end of the token
// every copy has landed (the barrier) and the next table is published.
#pragma once
#include <stdint.h>

#include <vector>

namespace moert {

constexpr double kHalfLife = 128.0;  // tokens

// log2 of each key's decayed value and the step of its last update; score = log2 v + step / (HALF_LIFE * layers).
struct Freq {
  std::vector<double> lv;
  std::vector<uint64_t> step;
  double per = 0;
  Freq() = default;
  Freq(int keys, int layers);
  void touch(int key, uint64_t s);
  double score(int key) const { return lv[key] + (double)step[key] / per; }
  void clear();
};

struct PlacementStats {
  uint64_t needed = 0, hits = 0, cpu = 0, copies = 0, dropped = 0, deferred = 0;
};

// A copy of host-store record `key` into pool slot `slot`, to be queued behind the work already queued.
struct CopyOrder {
  int slot, key;
};

class Placement {
 public:
  Placement(int layers, int experts, int top_k, int slots, int backlog);

  // Start of the first token: the table of the empty pool.
  void start();
  // Layer l of the current step: ids [m][top_k] (expert ids of each position, top-k order). Queues the copies held
  // for victims of layer l - 1, touches the frequency once per request, advances the step clock by m and counts the
  // requests. `union_keys` / `union_n` get the layer's keys in order of first appearance with their request counts,
  // `gpu` whether the token's table holds each (its slot is then table()[key]).
  void serve_layer(int l, const int* ids, int m, std::vector<int>* union_keys, std::vector<int>* union_n,
                   std::vector<char>* gpu);
  // After the host has computed the layer's missed experts: admissions for its keys that missed and have no slot
  // (in order of first appearance).
  void admit_layer();
  // End of the token: queues the copies held for the last layer; every copy has landed, so loading slots become
  // resident, and the next token's table is published.
  void end_token();

  const std::vector<int>& table() const { return table_; }  // key -> slot of the current token, -1 when absent
  std::vector<CopyOrder> take_copies();                      // the copies queued since the last call
  const PlacementStats& stats() const { return stats_; }
  int slots() const { return (int)slot_.size(); }
  int backlog() const { return backlog_; }
  int resident() const;
  double score(int key) const { return freq_.score(key); }

 private:
  enum Kind { FREE = 0, RESIDENT = 1, LOADING = 2, HELD = 3 };
  struct Slot {
    int kind = FREE, key = -1, after = -1;
  };
  int pending() const;
  void release_held(int layer);
  void publish();

  int L_, E_, K_, backlog_;
  std::vector<Slot> slot_;
  std::vector<int> key_slot_;  // key -> slot holding, loading or holding it, -1
  std::vector<uint64_t> version_;
  std::vector<int> table_;
  Freq freq_;
  uint64_t step_ = 0;
  int cur_layer_ = 0;
  std::vector<int> layer_keys_, misses_;
  std::vector<int> held_order_;  // held slots in the order of their admission
  std::vector<CopyOrder> copies_;
  PlacementStats stats_;
};

}  // namespace moert
