// Recording stand-in for libsq8's C ABI (include/sq8*.h) for CPU tests of host code that issues
// its launches (model::PagedBatchModel): each call appends one line, the function name and its
// arguments, to a log, with pointers numbered in order of first appearance (so two hosts that
// use their buffers in the same roles print the same log) and without the stream argument.
// Workspace queries return fixed sizes and the fused-epilogue queries a fixed rule (fused when
// M > 4 and N is even), restated by tests/test_native_scheduler.py for the Python model.
#include <cstdint>
#include <cstdio>
#include <iterator>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/sq8.h"
#include "../../include/sq8_batch.h"
#include "../../include/sq8_decode.h"
#include "hip/hip_runtime.h"

namespace {
struct Alloc {
  size_t bytes;
  int owned;  // allocated by the code under test (hipMalloc), not handed in
  int id;     // order of first appearance in the log, 0 = not yet
};
std::map<uintptr_t, Alloc> g_allocs;
int g_next_id = 0;
std::vector<std::string> g_log;

struct Line {
  std::ostringstream os;
  explicit Line(const char* name) { os << name; }
  // A pointer as p<allocation id>[+<byte offset>]; "?" outside every registered allocation.
  Line& p(const void* v) {
    if (!v) {
      os << " 0";
      return *this;
    }
    const uintptr_t a = reinterpret_cast<uintptr_t>(v);
    auto it = g_allocs.upper_bound(a);
    if (it == g_allocs.begin() || a >= std::prev(it)->first + std::prev(it)->second.bytes) {
      os << " ?";
      return *this;
    }
    --it;
    if (it->second.id == 0) it->second.id = ++g_next_id;
    os << " p" << it->second.id;
    if (a != it->first) os << "+" << (a - it->first);
    return *this;
  }
  Line& i(long long v) {
    os << " " << v;
    return *this;
  }
  Line& f(float v) {
    char b[32];
    std::snprintf(b, sizeof b, " %.6g", v);
    os << b;
    return *this;
  }
  ~Line() { g_log.push_back(os.str()); }
};
}  // namespace

hipError_t hipGraphLaunch(hipGraphExec_t, hipStream_t) {
  Line("graph_launch");
  return hipSuccess;
}
void mock_register(const void* p, size_t bytes, int owned) {
  g_allocs[reinterpret_cast<uintptr_t>(p)] = Alloc{bytes, owned, 0};
}
// The log, then "alloc p<id> <bytes>" for every allocation of the code under test that the
// log names, in id order.
void mock_print_log() {
  for (const std::string& s : g_log) std::printf("%s\n", s.c_str());
  std::map<int, size_t> sizes;
  for (const auto& a : g_allocs)
    if (a.second.owned && a.second.id) sizes[a.second.id] = a.second.bytes;
  for (const auto& s : sizes) std::printf("alloc p%d %zu\n", s.first, s.second);
}
void mock_mark(const char* what) { Line l(what); }

extern "C" {
const char* sq8_status_string(int) { return "mock"; }
int sq8_epilogue_fused(int M, int N, int, int) { return M > 4 && N % 2 == 0; }
int sq8_epilogue_packed_fused(int M, int N, int, int) { return M > 4 && N % 2 == 0; }
size_t sq8_epilogue_workspace_bytes(int, int, int, int, int) { return 4096; }
size_t sq8_epilogue_packed_workspace_bytes(int, int, int, int, int) { return 8192; }
size_t sq8_rmsnorm_rows_workspace_bytes(int, int, int, int, int) { return 4096; }
size_t sq8_rmsnorm_rows_packed_workspace_bytes(int, int, int, int, int) { return 8192; }
size_t sq8_paged_attention_workspace_bytes(int, int, int, int, int, int) { return 2048; }

int sq8_matmul(const float* x, const int8_t* w, const float* s, float* y, int M, int N, int K,
               int gs, void* ws, size_t wsb, void*) {
  Line("sq8_matmul").p(x).p(w).p(s).p(y).i(M).i(N).i(K).i(gs).p(ws).i(wsb);
  return 0;
}
int sq8_matmul_packed(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                      int K, int gs, void* ws, size_t wsb, void*) {
  Line("sq8_matmul_packed").p(x).p(w).p(s).p(y).i(M).i(N).i(K).i(gs).p(ws).i(wsb);
  return 0;
}
int sq8_matmul_epilogue(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                        int K, int gs, int epi, const float* r, void* ws, size_t wsb, void*) {
  Line("sq8_matmul_epilogue").p(x).p(w).p(s).p(y).i(M).i(N).i(K).i(gs).i(epi).p(r).p(ws).i(wsb);
  return 0;
}
int sq8_matmul_epilogue_packed(const float* x, const int8_t* w, const float* s, float* y, int M,
                               int N, int K, int gs, int epi, const float* r, void* ws,
                               size_t wsb, void*) {
  Line("sq8_matmul_epilogue_packed").p(x).p(w).p(s).p(y).i(M).i(N).i(K).i(gs).i(epi).p(r).p(ws)
      .i(wsb);
  return 0;
}
int sq8_matmul_rmsnorm_rows(float* x, const float* res, const float* nw, float eps,
                            const int8_t* w, const float* s, float* y, int M, int N, int K,
                            int gs, int epi, void* ws, size_t wsb, void*) {
  Line("sq8_matmul_rmsnorm_rows").p(x).p(res).p(nw).f(eps).p(w).p(s).p(y).i(M).i(N).i(K).i(gs)
      .i(epi).p(ws).i(wsb);
  return 0;
}
int sq8_matmul_rmsnorm_rows_packed(float* x, const float* res, const float* nw, float eps,
                                   const int8_t* w, const float* s, float* y, int M, int N,
                                   int K, int gs, int epi, void* ws, size_t wsb, void*) {
  Line("sq8_matmul_rmsnorm_rows_packed").p(x).p(res).p(nw).f(eps).p(w).p(s).p(y).i(M).i(N).i(K)
      .i(gs).i(epi).p(ws).i(wsb);
  return 0;
}
int sq8_embedding(const float* t, int vocab, int dim, const int32_t* tok, int n, float* out,
                  void*) {
  Line("sq8_embedding").p(t).i(vocab).i(dim).p(tok).i(n).p(out);
  return 0;
}
int sq8_rmsnorm(const float* x, const float* w, float* out, int rows, int dim, float eps, void*) {
  Line("sq8_rmsnorm").p(x).p(w).p(out).i(rows).i(dim).f(eps);
  return 0;
}
int sq8_add_rmsnorm(float* x, const float* r, const float* w, float* out, int rows, int dim,
                    float eps, void*) {
  Line("sq8_add_rmsnorm").p(x).p(r).p(w).p(out).i(rows).i(dim).f(eps);
  return 0;
}
int sq8_rope_tables(float* s, float* c, int hs, int max_seq, float theta, void*) {
  Line("sq8_rope_tables").p(s).p(c).i(hs).i(max_seq).f(theta);
  return 0;
}
int sq8_paged_rope_kv(float* qkv, int rows, int h, int kvh, int hs, const int32_t* pos,
                      const int32_t* tab, int stride, int bs, const float* sn, const float* cs,
                      float* kc, float* vc, void*) {
  Line("sq8_paged_rope_kv").p(qkv).i(rows).i(h).i(kvh).i(hs).p(pos).p(tab).i(stride).i(bs).p(sn)
      .p(cs).p(kc).p(vc);
  return 0;
}
int sq8_paged_attention(const float* qkv, int qs, int rows, int h, int kvh, int hs,
                        const int32_t* pos, const int32_t* tab, int stride, int bs,
                        const float* kc, const float* vc, float* out, void*) {
  Line("sq8_paged_attention").p(qkv).i(qs).i(rows).i(h).i(kvh).i(hs).p(pos).p(tab).i(stride)
      .i(bs).p(kc).p(vc).p(out);
  return 0;
}
int sq8_paged_attention_ws(const float* qkv, int qs, int rows, int h, int kvh, int hs,
                           const int32_t* pos, const int32_t* tab, int stride, int bs,
                           const float* kc, const float* vc, float* out, void* ws, size_t wsb,
                           void*) {
  Line("sq8_paged_attention_ws").p(qkv).i(qs).i(rows).i(h).i(kvh).i(hs).p(pos).p(tab).i(stride)
      .i(bs).p(kc).p(vc).p(out).p(ws).i(wsb);
  return 0;
}
int sq8_swiglu_rows(const float* gu, int rows, int ffn, float* out, void*) {
  Line("sq8_swiglu_rows").p(gu).i(rows).i(ffn).p(out);
  return 0;
}
size_t sq8_workspace_bytes(int, int, int, int) { return 4096; }
size_t sq8_argmax_workspace_bytes(int) { return 1024; }
size_t sq8_decode_attention_workspace_bytes(int, int, int) { return 2048; }
int sq8_matmul_rmsnorm(const float* x, const float* res, float* x_out, const float* nw, float eps,
                       const int8_t* w, const float* s, float* y, int N, int K, int gs, void*) {
  Line("sq8_matmul_rmsnorm").p(x).p(res).p(x_out).p(nw).f(eps).p(w).p(s).p(y).i(N).i(K).i(gs);
  return 0;
}
int sq8_matmul_rmsnorm_swiglu(const float* x, const float* res, float* x_out, const float* nw,
                              float eps, const int8_t* w, const float* s, float* y, int N, int K,
                              int gs, void*) {
  Line("sq8_matmul_rmsnorm_swiglu").p(x).p(res).p(x_out).p(nw).f(eps).p(w).p(s).p(y).i(N).i(K)
      .i(gs);
  return 0;
}
int sq8_rope_attention_decode(const float* qkv, int h, int kvh, int hs, const int32_t* pos,
                              const float* sn, const float* cs, float* kc, float* vc, float* out,
                              int max_seq, void*) {
  Line("sq8_rope_attention_decode").p(qkv).i(h).i(kvh).i(hs).p(pos).p(sn).p(cs).p(kc).p(vc)
      .p(out).i(max_seq);
  return 0;
}
int sq8_rope_attention_decode_ws(const float* qkv, int h, int kvh, int hs, const int32_t* pos,
                                 const float* sn, const float* cs, float* kc, float* vc,
                                 float* out, int max_seq, void* ws, size_t wsb, void*) {
  Line("sq8_rope_attention_decode_ws").p(qkv).i(h).i(kvh).i(hs).p(pos).p(sn).p(cs).p(kc).p(vc)
      .p(out).i(max_seq).p(ws).i(wsb);
  return 0;
}
int sq8_argmax_advance(const float* logits, int n, void* ws, size_t wsb, int32_t* pos,
                       int32_t* token, const float* emb, int vocab, int dim, float* x, void*) {
  Line("sq8_argmax_advance").p(logits).i(n).p(ws).i(wsb).p(pos).p(token).p(emb).i(vocab).i(dim)
      .p(x);
  return 0;
}
int sq8_step_advance(int32_t* pos, int32_t* token, const int32_t* next, void*) {
  Line("sq8_step_advance").p(pos).p(token).p(next);
  return 0;
}
size_t sq8_packed_weight_bytes(int N, int K) {
  return static_cast<size_t>((N + 15) / 16) * 16 * K;
}
// The packed layout computed on the host (byte 16 L + b of block (t, g) is w[16 t + L % 16]
// [64 g + 16 (L / 16) + b], rows past N zero), so that callers' arguments can be checked.
int sq8_pack_weights(const int8_t* w, int N, int K, int8_t* packed, void*) {
  Line("sq8_pack_weights").p(w).i(N).i(K).p(packed);
  const int T = (N + 15) / 16, G = K / 64;
  for (int t = 0; t < T; ++t)
    for (int g = 0; g < G; ++g)
      for (int L = 0; L < 64; ++L)
        for (int b = 0; b < 16; ++b) {
          const int row = 16 * t + L % 16, col = 64 * g + 16 * (L / 16) + b;
          packed[((static_cast<size_t>(t) * G + g) * 64 + L) * 16 + b] =
              row < N ? w[static_cast<size_t>(row) * K + col] : 0;
        }
  return 0;
}
int sq8_argmax_rows(const float* logits, int rows, int n, int32_t* out, void*) {
  Line("sq8_argmax_rows").p(logits).i(rows).i(n).p(out);
  return 0;
}
}  // extern "C"
