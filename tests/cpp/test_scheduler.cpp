// The C++ scheduler (scheduler::Scheduler, BlockAllocator, PrefixCache) on the CPU with a chain
// model: the value stored at a row's (physical block, offset) is chained from the value at
// position - 1 read back through the row's block table, as a transformer's KV depends on every
// earlier token, and a decode row's token is its stored value. Batched runs must therefore give
// every sequence the tokens of running it alone (or, when a pool too small for the set forces a
// sequence to finish early, a prefix of them). The model also checks that no row writes into a
// block another row references, that decode rows come first and that a sequence's prefill rows
// are in position order. Built with -fsanitize=address,undefined by tests/test_native_scheduler.py.
#include <algorithm>
#include <cstdio>
#include <map>
#include <memory>
#include <random>
#include <set>
#include <vector>

#include "scheduler/scheduler.h"
#include "test_util.h"

namespace {

struct ChainModel : scheduler::BatchModel {
  int bs = 16;
  const scheduler::BlockAllocator* alloc = nullptr;
  std::map<std::pair<int, int>, long long> kv;
  std::set<int> stop;
  int calls = 0;

  base::Status forward_batch(int batch, int nd, const int32_t* tokens, const int32_t* positions,
                             const int32_t* seq_ids, const int32_t* table, int stride,
                             int32_t* next) override {
    ++calls;
    for (int i = 0; i < batch; ++i) {
      const int32_t* t = table + static_cast<size_t>(i) * stride;
      const int p = positions[i];
      if (p / bs >= stride) return base::error::InvalidArgument("position beyond the table");
      const int blk = t[p / bs];
      EXPECT(blk >= 0, "position beyond the row's blocks");
      if (blk < 0) return base::error::InternalError("unmapped position");
      EXPECT(alloc->ref_count(blk) == 1, "write into a shared block");
      if (i > 0 && seq_ids[i] == seq_ids[i - 1] && i > nd)
        EXPECT(positions[i] == positions[i - 1] + 1, "prefill rows out of order");
      long long prev = 17;
      if (p > 0) {
        const auto it = kv.find({t[(p - 1) / bs], (p - 1) % bs});
        EXPECT(it != kv.end(), "reads a position never written");
        if (it != kv.end()) prev = it->second;
      }
      kv[{blk, p % bs}] = (prev * 1000033 + tokens[i] * 31LL + p) % 998244353;
    }
    for (int i = 0; i < nd; ++i) {
      const int32_t* t = table + static_cast<size_t>(i) * stride;
      next[i] = static_cast<int32_t>(kv[{t[positions[i] / bs], positions[i] % bs}] % 5000);
    }
    return base::error::Success();
  }
  bool is_sentence_ending(int32_t token) const override { return stop.count(token) != 0; }
};

struct Workload {
  std::vector<std::vector<int>> prompts;
  std::vector<int> arrival;  // step at which each prompt is added
  int max_batch, max_seq, max_gen, bs, num_blocks;
  bool prefix;
  std::set<int> stop;
};

Workload make(uint64_t seed) {
  std::mt19937_64 g(seed);
  auto uni = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(g); };
  Workload w;
  const int bss[] = {4, 8, 16};
  w.bs = bss[uni(0, 2)];
  std::vector<int> base(64);
  for (int& t : base) t = uni(0, 4999);
  const int n = uni(4, 13);
  int longest = 1;
  for (int i = 0; i < n; ++i) {
    const int len = uni(1, 59);
    std::vector<int> p;
    if (uni(0, 1)) {
      const int k = uni(0, len);
      p.assign(base.begin(), base.begin() + k);
    }
    while (static_cast<int>(p.size()) < len) p.push_back(uni(0, 4999));
    longest = std::max(longest, len);
    w.prompts.push_back(p);
    w.arrival.push_back(uni(0, 29));
  }
  w.max_gen = uni(1, 23);
  w.max_seq = longest + w.max_gen;
  w.max_batch = uni(1, 8);
  const int full = w.max_batch * ((w.max_seq + w.bs - 1) / w.bs);
  w.num_blocks = uni(0, 2) == 0 ? 0 : uni(std::min(full, std::max(4, full / 4)), full);
  w.prefix = uni(0, 9) < 7;
  const int nstop = uni(0, 39);
  for (int i = 0; i < nstop; ++i) w.stop.insert(uni(0, 4999));
  return w;
}

// Runs a workload; returns false when it did not finish within max_steps.
bool drive(const Workload& w, int only, std::map<int, std::vector<int>>* out,
           scheduler::Scheduler** keep, std::shared_ptr<ChainModel>* mkeep, int max_steps) {
  auto model = std::make_shared<ChainModel>();
  model->bs = w.bs;
  model->stop = w.stop;
  scheduler::SchedulerOptions opt;
  opt.num_blocks = only >= 0 ? 0 : w.num_blocks;
  opt.prefix_cache = only >= 0 ? false : w.prefix;
  auto* s = new scheduler::Scheduler(model, only >= 0 ? 1 : w.max_batch, w.max_seq, w.max_gen,
                                     w.bs, opt);
  model->alloc = &s->block_allocator();
  std::map<int, int> id_to_index;
  int step = 0;
  size_t added = 0;
  std::vector<int> order(w.prompts.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = static_cast<int>(i);
  std::stable_sort(order.begin(), order.end(),
                   [&](int a, int b) { return w.arrival[a] < w.arrival[b]; });
  while (added < order.size() || !s->all_finished()) {
    while (added < order.size() && (only >= 0 || w.arrival[order[added]] <= step)) {
      const int idx = order[added++];
      if (only >= 0 && idx != only) continue;
      const int id = s->add_request(w.prompts[idx]);
      EXPECT(id >= 0, "request refused");
      id_to_index[id] = idx;
    }
    ++step;
    if (s->all_finished()) continue;
    EXPECT(static_cast<bool>(s->step()), "step failed");
    EXPECT(s->block_allocator().invariant_holds(), "block pool invariant");
    if (step >= max_steps) break;
  }
  const bool done = s->all_finished();
  for (const scheduler::Sequence& q : s->get_finished())
    (*out)[id_to_index[q.id]] = q.generated_tokens;
  if (done) {
    EXPECT(s->block_allocator().free_block_count() == s->block_allocator().num_blocks(),
           "blocks not returned");
  }
  *keep = s;
  *mkeep = model;
  return done;
}

}  // namespace

int main() {
  int finished_runs = 0, preempting = 0, sharing = 0, stopping = 0;
  for (uint64_t seed = 0; seed < 300; ++seed) {
    const Workload w = make(seed);
    std::map<int, std::vector<int>> got;
    scheduler::Scheduler* s = nullptr;
    std::shared_ptr<ChainModel> m;
    const bool done = drive(w, -1, &got, &s, &m, 4000);
    preempting += s->preemptions() > 0;
    sharing += s->shared_prefix_blocks() > 0;
    delete s;
    if (!done) continue;
    ++finished_runs;
    for (size_t i = 0; i < w.prompts.size(); ++i) {
      std::map<int, std::vector<int>> alone;
      scheduler::Scheduler* s1 = nullptr;
      std::shared_ptr<ChainModel> m1;
      EXPECT(drive(w, static_cast<int>(i), &alone, &s1, &m1, 4000), "single run stalls");
      delete s1;
      const std::vector<int>& ref = alone[static_cast<int>(i)];
      const std::vector<int>& t = got[static_cast<int>(i)];
      EXPECT(t.size() <= ref.size() && std::equal(t.begin(), t.end(), ref.begin()),
             "batched tokens are not a prefix of the single-sequence run");
      if (!t.empty() && w.stop.count(t.back())) ++stopping;
    }
  }
  std::printf("runs finished %d / 300, with preemption %d, with shared prefixes %d, "
              "stop-token retirements %d\n", finished_runs, preempting, sharing, stopping);
  EXPECT(finished_runs > 250 && preempting > 20 && sharing > 20 && stopping > 0, "coverage");
  std::printf("scheduler: %d failure(s)\n", sq8test::failures());
  return sq8test::failures() == 0 ? 0 : 1;
}
