// Prints the libsq8 calls model::PagedBatchModel (or, in decoder mode, model::Int8Decoder) issues
// for a scripted run, built
// with g++ against host stand-ins of the HIP runtime (tests/cpp/mock_hip) and of libsq8
// (tests/cpp/mock_sq8.cpp). tests/test_native_scheduler.py compares the log with the calls the
// Python PagedBatchModel issues for the same steps.
//
// stdin, batch mode: "batch packed use_graphs split_kv", then per step "B nd", B tokens, B positions and
// B * table_stride block-table entries; "capture" instead of a step calls
// capture_decode_graphs(). Model: dim 64, FFN 96, 2 layers, 4 / 2 heads, vocab 50, 8 rows,
// max_seq 64, 40 blocks of 4. Decoder mode: "decoder use_graph split n_new n_prompt" and the
// prompt tokens (same model, max_seq 64).
#include <cstdio>
#include <cstdlib>
#include <iostream>
#include <string>
#include <vector>

#include "model/int8_decoder.h"
#include "model/paged_batch_model.h"

void mock_print_log();
void mock_mark(const char* what);
void mock_register(const void* p, size_t bytes, int owned);

int main() {
  std::string mode;
  int packed = 0, graphs = 0, split = 0;
  if (!(std::cin >> mode)) return 2;
  if (mode == "batch" && !(std::cin >> packed >> graphs >> split)) return 2;
  // mode "validate": forward_batch refuses bad rows before any launch.
  model::BatchModelConfig c;
  c.dim = 64;
  c.hidden_dim = 96;
  c.layer_num = 2;
  c.head_num = 4;
  c.kv_head_num = 2;
  c.vocab_size = 50;
  c.rope_theta = 1e6f;
  c.group_size = 64;
  std::vector<void*> bufs;
  auto fake = [&]() {  // a weight buffer handed in by the caller (not the model's own)
    bufs.push_back(std::malloc(64));
    mock_register(bufs.back(), 64, 0);
    return bufs.back();
  };
  model::BatchModelWeights w;
  // Allocation order mirrors the Python test's weight dict: per kind, per layer, (q, s).
  for (auto* v : {&w.qkv, &w.o, &w.gu, &w.down})
    for (int l = 0; l < c.layer_num; ++l)
      v->push_back({static_cast<const int8_t*>(fake()), static_cast<const float*>(fake())});
  w.cls = {static_cast<const int8_t*>(fake()), static_cast<const float*>(fake())};
  w.embedding = static_cast<const float*>(fake());
  for (int i = 0; i < 2 * c.layer_num + 1; ++i) w.norm.push_back(static_cast<const float*>(fake()));
  w.packed = packed != 0;
  if (mode == "decoder") {
    int use_graph = 0, n_new = 0, np = 0;
    std::cin >> use_graph >> split >> n_new >> np;
    std::vector<int32_t> prompt(np), out;
    for (auto& t : prompt) std::cin >> t;
    model::Int8Decoder dec(c, w, 64, nullptr, split != 0);
    base::Status st = dec.init();
    if (st) st = dec.generate(prompt, n_new, &out, use_graph != 0);
    if (!st) {
      std::printf("decoder failed: %s\n", st.get_err_msg().c_str());
      return 1;
    }
    mock_print_log();
    for (void* p : bufs) std::free(p);
    return 0;
  }
  if (mode == "validate") {  // host-side refusals: nothing may reach libsq8
    model::PagedBatchModel m(c, w, 8, 64, 40, 4, nullptr, true, true);
    if (!m.init()) return 1;
    const int S = m.max_blocks_per_seq();
    std::vector<int32_t> tab(8 * S, -1), next(8);
    tab[0] = 3;  // row 0 holds block 3 at index 0 only
    int32_t tok[8] = {1, 2, 3, 4, 5, 6, 7, 8}, pos[8] = {0};
    struct Case {
      const char* what;
      int B, nd, stride, pos0, tok0;
    } cases[] = {{"no rows", 0, 0, S, 0, 1},          {"too many rows", 9, 0, S, 0, 1},
                 {"decode rows > rows", 1, 2, S, 0, 1}, {"table width", 1, 1, S - 1, 0, 1},
                 {"position past max_seq", 1, 1, S, 64, 1},
                 {"unmapped block", 1, 1, S, 4, 1},     {"token id", 1, 1, S, 0, 50},
                 {"negative token", 1, 1, S, 0, -1}};
    int failures = 0;
    for (const Case& k : cases) {
      pos[0] = k.pos0;
      tok[0] = k.tok0;
      const base::Status st = m.forward_batch(k.B, k.nd, tok, pos, nullptr, tab.data(),
                                              k.stride, next.data());
      std::printf("%s: %s\n", k.what, st ? "accepted" : st.get_err_msg().c_str());
      failures += static_cast<bool>(st);
    }
    mock_print_log();  // only the rope tables of init()
    for (void* p : bufs) std::free(p);
    return failures;
  }
  model::PagedBatchModel m(c, w, 8, 64, 40, 4, nullptr, graphs != 0, split != 0);
  base::Status st = m.init();
  if (!st) {
    std::printf("init failed: %s\n", st.get_err_msg().c_str());
    return 1;
  }
  const int stride = m.max_blocks_per_seq();
  std::string word;
  while (std::cin >> word) {
    if (word == "capture") {
      mock_mark("capture_decode_graphs");
      st = m.capture_decode_graphs();
      if (!st) {
        std::printf("capture failed: %s\n", st.get_err_msg().c_str());
        return 1;
      }
      continue;
    }
    const int B = std::atoi(word.c_str());
    int nd = 0;
    std::cin >> nd;
    std::vector<int32_t> tok(B), pos(B), tab(static_cast<size_t>(B) * stride), next(B);
    for (auto& t : tok) std::cin >> t;
    for (auto& p : pos) std::cin >> p;
    for (auto& t : tab) std::cin >> t;
    mock_mark("step");
    st = m.forward_batch(B, nd, tok.data(), pos.data(), nullptr, tab.data(), stride, next.data());
    if (!st) {
      std::printf("step failed: %s\n", st.get_err_msg().c_str());
      return 1;
    }
  }
  mock_print_log();
  for (void* p : bufs) std::free(p);
  return 0;
}
