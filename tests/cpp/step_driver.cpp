// A C++ caller of libfeattn.so shaped like the reference's model runner
// (src/cuda_model.cpp): graph buckets (common.cpp:45-51; the smallest bucket
// that holds the batch gets a plan and a captured graph, :118, :150-157),
// the FIFO page allocator with its prefix cache (scheduler.cpp:5-36), the
// per-step metadata (:131-142), and per layer the q/k RMSNorm + RoPE + paged
// append followed by paged attention (:91-96), all through the reference's
// fe::cuda:: signatures (include/fe_native_hip.hpp).  Prefill steps run
// eagerly: the prompts, then a request whose prompt starts with a published
// prefix and computes only the rest over the shared pages; decode steps
// replay a HIP graph captured once on the bucket's fixed buffers, with
// prepare_plan called outside the capture as the reference does.
//
// Inputs are generated here from a fixed seed; every input and output is
// written to one file so that a test can replay the same sequence on the
// oracle:  step_driver <output file>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "fe_attn.h"
#include "fe_driver.h"
#include "fe_native_hip.hpp"
#include "fe_ops.h"

namespace {

constexpr int kHq = 32, kHkv = 8, kDim = 128, kPage = 16, kPool = 64, kMaxLen = 256, kLayers = 2;
constexpr int kMaxSeqs = 4;
constexpr int kQkv = (kHq + 2 * kHkv) * kDim;  // elements of one projection row
constexpr float kEps = 1e-6f;

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
void fe_check(int rc, const char* what) {
  if (rc != FE_OK) throw std::runtime_error(std::string(what) + ": " + fe_attn_last_error());
}

// xorshift64*; values are rounded to bf16 (nearest even) from uniform [-2, 2).
struct Rng {
  uint64_t s;
  uint32_t next() {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return (uint32_t)((s * 2685821657736338717ull) >> 32);
  }
  uint16_t bf16() {
    const float f = ((float)next() / 4294967296.0f) * 4.0f - 2.0f;
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  }
};

// Output file: "FESTEP01", then records {u32 name length, name, u32 dtype
// (0 u16, 1 i32, 2 i64, 3 f32), u32 ndim, u64 dims[ndim], data}.
struct Writer {
  FILE* f;
  explicit Writer(const char* path) : f(std::fopen(path, "wb")) {
    if (!f) throw std::runtime_error("cannot open output file");
    std::fwrite("FESTEP01", 1, 8, f);
  }
  ~Writer() { std::fclose(f); }
  void put(const std::string& name, uint32_t dtype, std::vector<uint64_t> dims, const void* data, size_t bytes) {
    const uint32_t n = (uint32_t)name.size(), nd = (uint32_t)dims.size();
    std::fwrite(&n, 4, 1, f);
    std::fwrite(name.data(), 1, n, f);
    std::fwrite(&dtype, 4, 1, f);
    std::fwrite(&nd, 4, 1, f);
    std::fwrite(dims.data(), 8, nd, f);
    std::fwrite(data, 1, bytes, f);
  }
  template <typename T>
  void vec(const std::string& name, uint32_t dtype, const std::vector<T>& v) {
    put(name, dtype, {(uint64_t)v.size()}, v.data(), v.size() * sizeof(T));
  }
  void device16(const std::string& name, std::vector<uint64_t> dims, const void* dptr) {
    size_t n = 1;
    for (uint64_t d : dims) n *= d;
    std::vector<uint16_t> h(n);
    hip_check(hipMemcpy(h.data(), dptr, n * 2, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    put(name, 0, dims, h.data(), n * 2);
  }
};

template <typename T>
T* dalloc(size_t n) {
  void* p = nullptr;
  hip_check(hipMalloc(&p, n * sizeof(T)), "hipMalloc");
  hip_check(hipMemset(p, 0, n * sizeof(T)), "hipMemset");
  return static_cast<T*>(p);
}

struct Seq {
  int64_t id;
  int64_t length;  // tokens in the cache after the step
};

// The per-step host metadata for `seqs` (start, rows each) padded to
// `count` entries of `entry_rows` rows, as CudaModel::prepare builds it.
struct Meta {
  std::vector<int64_t> positions, slots;
  std::vector<int32_t> qo, kv, pages, last;
};

Meta metadata(fe_blocks* blocks, const std::vector<Seq>& seqs, const std::vector<int64_t>& start,
              const std::vector<int32_t>& rows, int count, int entry_rows) {
  std::vector<int32_t> off{0}, tables;
  for (const Seq& s : seqs) {
    int n = 0;
    fe_check(fe_blocks_table(blocks, s.id, nullptr, 0, &n), "fe_blocks_table");
    std::vector<int32_t> t(n);
    fe_check(fe_blocks_table(blocks, s.id, t.data(), n, &n), "fe_blocks_table");
    tables.insert(tables.end(), t.begin(), t.end());
    off.push_back((int32_t)tables.size());
  }
  int nr = 0, np = 0;
  const int n = (int)seqs.size();
  fe_check(fe_prepare_metadata(n, start.data(), rows.data(), off.data(), tables.data(), count, entry_rows, kPage,
                               kMaxLen, kPool, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0, nullptr, &nr, &np),
           "fe_prepare_metadata (sizes)");
  Meta m;
  m.positions.resize(nr);
  m.slots.resize(nr);
  m.qo.resize(count + 1);
  m.kv.resize(count + 1);
  m.pages.resize(np);
  m.last.resize(count);
  fe_check(fe_prepare_metadata(n, start.data(), rows.data(), off.data(), tables.data(), count, entry_rows, kPage,
                               kMaxLen, kPool, m.positions.data(), m.slots.data(), nr, m.qo.data(), m.kv.data(),
                               m.pages.data(), np, m.last.data(), &nr, &np),
           "fe_prepare_metadata");
  return m;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: step_driver <output file>\n");
    return 2;
  }
  try {
    Writer out(argv[1]);
    Rng rng{0x9e3779b97f4a7c15ull};
    hipStream_t st;
    hip_check(hipStreamCreate(&st), "hipStreamCreate");

    // model state: per-layer q/k norm weights and KV caches, the RoPE table
    const size_t cache_elems = (size_t)(kPool + 1) * kPage * kHkv * kDim;
    std::vector<uint16_t*> kc(kLayers), vc(kLayers), qn(kLayers), kn(kLayers);
    for (int l = 0; l < kLayers; ++l) {
      kc[l] = dalloc<uint16_t>(cache_elems);
      vc[l] = dalloc<uint16_t>(cache_elems);
      std::vector<uint16_t> w(kDim), u(kDim);
      for (auto& x : w) x = rng.bf16();
      for (auto& x : u) x = rng.bf16();
      qn[l] = dalloc<uint16_t>(kDim);
      kn[l] = dalloc<uint16_t>(kDim);
      hip_check(hipMemcpy(qn[l], w.data(), kDim * 2, hipMemcpyHostToDevice), "hipMemcpy");
      hip_check(hipMemcpy(kn[l], u.data(), kDim * 2, hipMemcpyHostToDevice), "hipMemcpy");
      out.vec("qn" + std::to_string(l), 0, w);
      out.vec("kn" + std::to_string(l), 0, u);
    }
    float* table = dalloc<float>((size_t)kMaxLen * kDim);
    fe_check(fe_rope_table(table, kMaxLen, kDim, 1e6, st), "fe_rope_table");
    {
      std::vector<float> t((size_t)kMaxLen * kDim);
      hip_check(hipMemcpy(t.data(), table, t.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy");
      out.put("rope_table", 3, {(uint64_t)kMaxLen, (uint64_t)kDim}, t.data(), t.size() * 4);
    }

    // graph buckets (cuda_model.cpp:150-157 capture one graph per bucket)
    int nb = 0;
    fe_check(fe_graph_buckets(kMaxSeqs, nullptr, 0, &nb), "fe_graph_buckets");
    std::vector<int64_t> buckets(nb);
    fe_check(fe_graph_buckets(kMaxSeqs, buckets.data(), nb, &nb), "fe_graph_buckets");
    out.vec("buckets", 2, buckets);
    fe_blocks* blocks = nullptr;
    fe_check(fe_blocks_create_ex(kPool, kPage, 1, &blocks), "fe_blocks_create_ex");

    std::vector<Seq> seqs = {{1, 40}, {2, 5}, {3, 17}};
    const int n = (int)seqs.size();

    // One prefill step run eagerly with a plan sized for it: metadata, then
    // per layer the fused norm + RoPE + append and the attention; every
    // input and output is recorded under `tag`.
    auto eager_step = [&](const std::string& tag, const std::vector<Seq>& ss, const std::vector<int64_t>& start,
                          const std::vector<int32_t>& rows) {
      const int ns = (int)ss.size();
      Meta m = metadata(blocks, ss, start, rows, ns, 0);
      const int R = (int)m.positions.size();
      fe::cuda::AttentionPlan* plan = fe::cuda::create_plan(kHq, kHkv, kDim, kPage, kMaxSeqs, kMaxLen / kPage + 1,
                                                            true, kPool);
      fe::cuda::prepare_plan(plan, m.qo.data(), m.kv.data(), m.pages.data(), m.last.data(), ns, R, false, st);
      int64_t* pos = dalloc<int64_t>(R);
      int64_t* slots = dalloc<int64_t>(R);
      hip_check(hipMemcpy(pos, m.positions.data(), R * 8, hipMemcpyHostToDevice), "hipMemcpy");
      hip_check(hipMemcpy(slots, m.slots.data(), R * 8, hipMemcpyHostToDevice), "hipMemcpy");
      uint16_t* qkv = dalloc<uint16_t>((size_t)R * kQkv);
      uint16_t* q = dalloc<uint16_t>((size_t)R * kHq * kDim);
      uint16_t* o = dalloc<uint16_t>((size_t)R * kHq * kDim);
      out.vec(tag + "_qo", 1, m.qo);
      out.vec(tag + "_kv", 1, m.kv);
      out.vec(tag + "_pages", 1, m.pages);
      out.vec(tag + "_last", 1, m.last);
      out.vec(tag + "_positions", 2, m.positions);
      out.vec(tag + "_slots", 2, m.slots);
      for (int l = 0; l < kLayers; ++l) {
        std::vector<uint16_t> x((size_t)R * kQkv);
        for (auto& v : x) v = rng.bf16();
        hip_check(hipMemcpy(qkv, x.data(), x.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
        fe::cuda::norm_rope_store(qkv, kQkv, qn[l], kn[l], kEps, q, kc[l], vc[l], pos, slots, table, R, kHq, kHkv,
                                  kDim, true, st, kMaxLen, (kPool + 1) * kPage);
        fe::cuda::attention(plan, q, kc[l], vc[l], o, true, st);
        hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
        const std::string p = tag + "_l" + std::to_string(l) + "_";
        out.vec(p + "qkv", 0, x);
        out.device16(p + "q", {(uint64_t)R, kHq, kDim}, q);
        out.device16(p + "out", {(uint64_t)R, kHq, kDim}, o);
      }
      fe::cuda::destroy_plan(plan);
      (void)hipFree(pos);
      (void)hipFree(slots);
      (void)hipFree(qkv);
      (void)hipFree(q);
      (void)hipFree(o);
    };
    auto table_of = [&](int64_t id) {
      int k = 0;
      fe_check(fe_blocks_table(blocks, id, nullptr, 0, &k), "fe_blocks_table");
      std::vector<int32_t> t(k);
      fe_check(fe_blocks_table(blocks, id, t.data(), k, &k), "fe_blocks_table");
      return t;
    };

    // token ids of the prompts (only the prefix cache reads them)
    std::vector<std::vector<int64_t>> tokens(n);
    for (int i = 0; i < n; ++i) {
      for (int64_t t = 0; t < seqs[i].length; ++t) tokens[i].push_back((int64_t)(rng.next() % 1000));
      out.vec("tokens" + std::to_string(seqs[i].id), 2, tokens[i]);
    }

    // ---- step 0: prefill of the prompts (nothing is published yet, so the
    // probes find nothing), then their full pages are published
    {
      std::vector<int64_t> start(n, 0);
      std::vector<int32_t> rows(n);
      for (int i = 0; i < n; ++i) {
        int64_t cached = -1;
        fe_check(fe_blocks_probe(blocks, seqs[i].id, tokens[i].data(), seqs[i].length, &cached), "fe_blocks_probe");
        if (cached != 0) throw std::runtime_error("empty prefix cache reported a hit");
        rows[i] = (int32_t)seqs[i].length;
        int ok = 0;
        fe_check(fe_blocks_ensure(blocks, seqs[i].id, seqs[i].length, &ok), "fe_blocks_ensure");
        if (!ok) throw std::runtime_error("page pool exhausted");
      }
      eager_step("s0", seqs, start, rows);
      for (int i = 0; i < n; ++i)
        fe_check(fe_blocks_publish(blocks, seqs[i].id, tokens[i].data(), seqs[i].length, seqs[i].length),
                 "fe_blocks_publish");
    }

    // ---- a request whose first 36 tokens are sequence 1's: the probe hands
    // it sequence 1's two full pages (32 tokens), and it computes its last 8
    // rows into a page of its own over them; it finishes after this step
    {
      Seq late{4, 40};
      std::vector<int64_t> t4(tokens[0].begin(), tokens[0].begin() + 36);
      for (int k = 0; k < 4; ++k) t4.push_back((int64_t)(rng.next() % 1000));
      out.vec("tokens4", 2, t4);
      int64_t cached = -1;
      fe_check(fe_blocks_probe(blocks, late.id, t4.data(), late.length, &cached), "fe_blocks_probe");
      int ok = 0;
      fe_check(fe_blocks_ensure(blocks, late.id, late.length, &ok), "fe_blocks_ensure");
      if (!ok) throw std::runtime_error("page pool exhausted");
      const std::vector<int32_t> t = table_of(late.id), t1 = table_of(seqs[0].id);
      if (cached != 32 || t.size() != 3 || t[0] != t1[0] || t[1] != t1[1] || t[2] == t1[2])
        throw std::runtime_error("prefix cache did not share sequence 1's pages");
      out.vec("p_cached", 2, std::vector<int64_t>{cached});
      eager_step("p", {late}, {cached}, {(int32_t)(late.length - cached)});
      fe_check(fe_blocks_forget(blocks, late.id), "fe_blocks_forget");
      fe_prefix_stats ps{};
      fe_check(fe_blocks_prefix_stats(blocks, &ps), "fe_blocks_prefix_stats");
      out.vec("prefix_stats", 2,
              std::vector<int64_t>{ps.requests, ps.hit_requests, ps.cached_blocks, ps.new_blocks, ps.resident_blocks,
                                   ps.evictions});
      std::printf("prefix step done (cached %lld)\n", (long long)cached);
      std::fflush(stdout);
    }

    // ---- decode steps through the graph of the smallest bucket >= n
    int64_t bucket = 0;
    for (int64_t b : buckets)
      if (b >= n) {
        bucket = b;
        break;
      }
    if (bucket == 0) throw std::runtime_error("no graph bucket");
    const int B = (int)bucket;
    fe::cuda::AttentionPlan* plan = fe::cuda::create_plan(kHq, kHkv, kDim, kPage, B, kMaxLen / kPage + 1, true, kPool);
    int64_t* pos = dalloc<int64_t>(B);
    int64_t* slots = dalloc<int64_t>(B);
    uint16_t* qkv = dalloc<uint16_t>((size_t)kLayers * B * kQkv);  // fixed input buffer of the entry
    uint16_t* q = dalloc<uint16_t>((size_t)B * kHq * kDim);
    uint16_t* o = dalloc<uint16_t>((size_t)kLayers * B * kHq * kDim);
    auto body = [&]() {
      for (int l = 0; l < kLayers; ++l) {
        fe::cuda::norm_rope_store(qkv + (size_t)l * B * kQkv, kQkv, qn[l], kn[l], kEps, q, kc[l], vc[l], pos, slots,
                                  table, B, kHq, kHkv, kDim, true, st, kMaxLen, (kPage) * (kPool + 1));
        fe::cuda::attention(plan, q, kc[l], vc[l], o + (size_t)l * B * kHq * kDim, true, st);
      }
    };
    hipGraphExec_t exec = nullptr;
    const int steps = 3;
    for (int step = 1; step <= steps; ++step) {
      std::vector<int64_t> start(n);
      std::vector<int32_t> rows(n, 1);
      for (int i = 0; i < n; ++i) {
        start[i] = seqs[i].length;
        seqs[i].length += 1;
        int ok = 0;
        fe_check(fe_blocks_ensure(blocks, seqs[i].id, seqs[i].length, &ok), "fe_blocks_ensure");
        if (!ok) throw std::runtime_error("page pool exhausted");
      }
      Meta m = metadata(blocks, seqs, start, rows, B, 1);
      std::vector<uint16_t> x((size_t)kLayers * B * kQkv);
      for (auto& v : x) v = rng.bf16();
      // fixed-address inputs first, then prepare outside any capture
      hip_check(hipMemcpy(qkv, x.data(), x.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
      hip_check(hipMemcpy(pos, m.positions.data(), B * 8, hipMemcpyHostToDevice), "hipMemcpy");
      hip_check(hipMemcpy(slots, m.slots.data(), B * 8, hipMemcpyHostToDevice), "hipMemcpy");
      fe::cuda::prepare_plan(plan, m.qo.data(), m.kv.data(), m.pages.data(), m.last.data(), B, B, true, st);
      if (exec == nullptr) {
        // the reference runs the body eagerly before capturing it
        // (cuda_model.cpp:153); here the eager run is the first decode step
        body();
        hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
        hipGraph_t graph;
        hip_check(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal), "hipStreamBeginCapture");
        body();
        hip_check(hipStreamEndCapture(st, &graph), "hipStreamEndCapture");
        hip_check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
        hip_check(hipGraphDestroy(graph), "hipGraphDestroy");
      } else {
        hip_check(hipGraphLaunch(exec, st), "hipGraphLaunch");
      }
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
      const std::string p = "s" + std::to_string(step) + "_";
      out.vec(p + "qo", 1, m.qo);
      out.vec(p + "kv", 1, m.kv);
      out.vec(p + "pages", 1, m.pages);
      out.vec(p + "last", 1, m.last);
      out.vec(p + "positions", 2, m.positions);
      out.vec(p + "slots", 2, m.slots);
      out.vec(p + "qkv", 0, x);
      out.device16(p + "out", {(uint64_t)kLayers, (uint64_t)B, kHq, kDim}, o);
      std::printf("decode step %d done (bucket %d)\n", step, B);
      std::fflush(stdout);
    }
    for (int l = 0; l < kLayers; ++l) {
      out.device16("final_kc" + std::to_string(l), {(uint64_t)(kPool + 1) * kPage, kHkv, kDim}, kc[l]);
      out.device16("final_vc" + std::to_string(l), {(uint64_t)(kPool + 1) * kPage, kHkv, kDim}, vc[l]);
    }
    hip_check(hipGraphExecDestroy(exec), "hipGraphExecDestroy");
    fe::cuda::destroy_plan(plan);
    for (const Seq& s : seqs) fe_check(fe_blocks_release(blocks, s.id), "fe_blocks_release");
    if (fe_blocks_used(blocks) != 0) throw std::runtime_error("pages leaked");
    fe_check(fe_blocks_destroy(blocks), "fe_blocks_destroy");
    std::printf("ok\n");
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "step_driver: %s\n", e.what());
    return 1;
  }
}
