// llm-runner: the native generation runner over libq4llm (the MI355X counterpart of the
// reference's runner/llm_runner.c, which drives IREE-compiled LlamaQ4 modules on Adreno).
//
//   llm-runner --weights=model.q4w --prompt=ids.txt [--max_new_tokens=32] [--chunk=128]
//              [--buckets=256,512,1024,2048,4096] [--schedule=bucketed|max] [--n_layers=N]
//              [--n_kv_heads=N] [--head_dim=N] [--max_ctx=N] [--stop_ids=a,b] [--warmup=1] [--plan]
//              [--decode_steps=8]
//
// Kept from llm_runner.c (same flag names and meaning, same schedule, same JSON keys):
//   * prefill in chunks of --chunk tokens, the last chunk zero-padded, last = n - 1 of the chunk;
//     bucket = smallest compiled bucket >= start + chunk (llm_runner.c:143-149, 210-222);
//   * the first generated token comes from prefill; decode at pos = n_prompt, ... with the bucket
//     >= pos + 1 until --max_new_tokens exist or a stop id appears (:226-245);
//   * --schedule=max always uses the largest bucket (:18-19, 143-144);
//   * the runner owns the zeroed KV caches for the whole run and the steps write them in place
//     (:301-315);
//   * warm-up: every entry point the schedule will use runs --warmup times before timing (:175-203);
//   * errors (empty prompt, prompt + new > max_ctx, no bucket) print to stderr and exit 1 (:327-331);
//   * one JSON object on stdout (:249-262).
// In place of the IREE module + parameter archive, the weights come from a packed-weight file
// (q4llm/packed.py) copied once to HBM, and each entry point prefill_c{C}_l{L} / decode_l{L} is one
// q4llm_step captured into a HIP graph on first use and replayed; per call the host copies the
// token ids, start and last into pinned buffers, launches the graph and reads back 4 bytes.
// --decode_steps=K (default 8; 1 = one step per launch): while K more tokens fit in --max_new_tokens
// and in the current bucket, one graph of K self-feeding decode steps runs per launch and the host
// reads the K tokens back at once; tokens after a stop id are dropped (their steps only wrote cache
// rows past the end of the sequence), so the output is that of one step per launch.
// --plan prints the schedule (the buckets of every prefill chunk and decode step) and exits
// without touching the GPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "q4llm.h"

namespace {

struct Flags {
  std::string weights, prompt, buckets = "256,512,1024,2048,4096", schedule = "bucketed", stop_ids;
  int max_new_tokens = 32, chunk = 128, n_layers = -1, n_kv_heads = -1, head_dim = -1, max_ctx = -1, warmup = 1;
  int decode_steps = 8;
  bool plan = false;
};

[[noreturn]] __attribute__((format(printf, 1, 2))) void die(const char* fmt, ...) {
  std::fprintf(stderr, "llm-runner: ");
  va_list ap;
  va_start(ap, fmt);
  std::vfprintf(stderr, fmt, ap);
  va_end(ap);
  std::fprintf(stderr, "\n");
  std::exit(1);
}

#define HIP_OK(expr)                                                                               \
  do {                                                                                             \
    hipError_t e_ = (expr);                                                                        \
    if (e_ != hipSuccess) {                                                                        \
      std::fprintf(stderr, "llm-runner: %s failed: %s\n", #expr, hipGetErrorString(e_));           \
      std::exit(1);                                                                                \
    }                                                                                              \
  } while (0)

#define Q4_OK_OR_DIE(expr)                                                                         \
  do {                                                                                             \
    int st_ = (expr);                                                                              \
    if (st_ != Q4_OK) {                                                                            \
      std::fprintf(stderr, "llm-runner: %s -> %s (hipError %d)\n", #expr, q4llm_status_string(st_), \
                   q4llm_last_hip_error());                                                        \
      std::exit(1);                                                                                \
    }                                                                                              \
  } while (0)

double now_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// Whitespace/comma separated integers, as parse_ints in llm_runner.c:55-65 (non-numbers skipped).
std::vector<int32_t> parse_ints(const std::string& s) {
  std::vector<int32_t> out;
  const char* p = s.c_str();
  while (*p) {
    char* end = nullptr;
    const long v = std::strtol(p, &end, 10);
    if (end == p) {
      ++p;
      continue;
    }
    out.push_back(static_cast<int32_t>(v));
    p = end;
  }
  return out;
}

Flags parse_flags(int argc, char** argv) {
  Flags f;
  for (int i = 1; i < argc; ++i) {
    std::string a = argv[i];
    if (a.rfind("--", 0) != 0) die("unexpected argument %s", argv[i]);
    a = a.substr(2);
    std::string key = a, val;
    const size_t eq = a.find('=');
    if (eq != std::string::npos) {
      key = a.substr(0, eq);
      val = a.substr(eq + 1);
    } else if (key != "plan") {
      if (i + 1 >= argc) die("flag --%s needs a value", key.c_str());
      val = argv[++i];
    }
    auto num = [&](int* dst) { *dst = std::atoi(val.c_str()); };
    if (key == "weights") f.weights = val;
    else if (key == "prompt") f.prompt = val;
    else if (key == "buckets") f.buckets = val;
    else if (key == "schedule") f.schedule = val;
    else if (key == "stop_ids") f.stop_ids = val;
    else if (key == "max_new_tokens") num(&f.max_new_tokens);
    else if (key == "chunk") num(&f.chunk);
    else if (key == "n_layers") num(&f.n_layers);
    else if (key == "n_kv_heads") num(&f.n_kv_heads);
    else if (key == "head_dim") num(&f.head_dim);
    else if (key == "max_ctx") num(&f.max_ctx);
    else if (key == "warmup") num(&f.warmup);
    else if (key == "decode_steps") num(&f.decode_steps);
    else if (key == "plan") f.plan = val.empty() || val == "1" || val == "true";
    else die("unknown flag --%s", key.c_str());
  }
  if (f.schedule != "bucketed" && f.schedule != "max") die("--schedule must be bucketed or max, not %s", f.schedule.c_str());
  if (f.chunk <= 0) die("--chunk must be positive");
  if (f.decode_steps <= 0) die("--decode_steps must be positive");
  return f;
}

// Smallest bucket >= needed, the largest under schedule max, -1 if none (llm_runner.c:143-149).
int pick_bucket(const std::vector<int32_t>& buckets, int needed, bool use_max) {
  if (use_max) return buckets.back();
  for (int b : buckets)
    if (b >= needed) return b;
  return -1;
}

struct Plan {
  std::vector<int> prefill, decode;  // bucket of every prefill chunk and of every possible decode step
};

Plan make_plan(int n_prompt, int max_new, int C, const std::vector<int32_t>& buckets, int max_ctx, bool use_max) {
  if (n_prompt == 0) die("empty prompt");
  const int total = n_prompt + max_new;
  if (total > max_ctx || ((n_prompt + C - 1) / C) * C > max_ctx)
    die("prompt %d + new %d exceeds max_ctx %d", n_prompt, max_new, max_ctx);
  Plan p;
  for (int start = 0; start < n_prompt; start += C) {
    const int L = pick_bucket(buckets, start + C, use_max);
    if (L < 0) die("no bucket >= %d", start + C);
    p.prefill.push_back(L);
  }
  for (int pos = n_prompt; pos < total - 1; ++pos) p.decode.push_back(pick_bucket(buckets, pos + 1, use_max));
  return p;
}

std::string read_file(const std::string& path) {
  FILE* fp = std::fopen(path.c_str(), "rb");
  if (!fp) die("cannot open --prompt=%s", path.c_str());
  std::string s;
  char buf[65536];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof buf, fp)) > 0) s.append(buf, n);
  std::fclose(fp);
  return s;
}

// ------------------------------------------------------------------------------------------------
// Packed-weight file (layout in q4llm/packed.py): ASCII header, then 256-byte aligned tensors.
// ------------------------------------------------------------------------------------------------

struct TensorMeta {
  std::string dtype;
  uint64_t offset = 0, nbytes = 0;
  std::vector<int64_t> shape;
};

struct Packed {
  std::map<std::string, long> ints;
  float eps = 0.0f;
  std::map<std::string, TensorMeta> tensors;
  std::vector<void*> device_buffers;
  std::map<std::string, void*> dev;
};

void load_packed(const std::string& path, Packed* pk) {
  FILE* fp = std::fopen(path.c_str(), "rb");
  if (!fp) die("cannot open --weights=%s", path.c_str());
  std::string head(1 << 20, '\0');
  head.resize(std::fread(&head[0], 1, head.size(), fp));
  const size_t end = head.find("\nend\n");
  if (head.rfind("Q4LLM-PACKED 1\n", 0) != 0 || end == std::string::npos) die("%s is not a packed-weight file", path.c_str());
  size_t pos = head.find('\n') + 1;
  while (pos <= end) {
    const size_t nl = head.find('\n', pos);
    const std::string line = head.substr(pos, nl - pos);
    pos = nl + 1;
    char kind[16] = {0}, name[256] = {0}, dt[8] = {0}, val[64] = {0};
    if (std::sscanf(line.c_str(), "%15s", kind) != 1) continue;
    if (!std::strcmp(kind, "config")) {
      if (std::sscanf(line.c_str(), "%*s %255s %63s", name, val) != 2) die("bad header line: %s", line.c_str());
      if (!std::strcmp(name, "eps")) pk->eps = std::strtof(val, nullptr);
      else pk->ints[name] = std::strtol(val, nullptr, 10);
    } else if (!std::strcmp(kind, "tensor")) {
      unsigned long long off = 0, nb = 0;
      int nd = 0, used = 0;
      if (std::sscanf(line.c_str(), "%*s %255s %7s %llu %llu %d%n", name, dt, &off, &nb, &nd, &used) != 5)
        die("bad tensor line: %s", line.c_str());
      TensorMeta m;
      m.dtype = dt;
      m.offset = off;
      m.nbytes = nb;
      const char* q = line.c_str() + used;
      for (int d = 0; d < nd; ++d) {
        char* e = nullptr;
        m.shape.push_back(std::strtoll(q, &e, 10));
        q = e;
      }
      pk->tensors[name] = m;
    } else if (!std::strcmp(kind, "end")) {
      break;
    } else {
      die("bad header line: %s", line.c_str());
    }
  }
  for (const char* k : {"dim", "n_layers", "n_heads", "n_kv", "head_dim", "inter", "vocab", "group", "max_ctx"})
    if (!pk->ints.count(k)) die("%s: header lacks config %s", path.c_str(), k);
  std::vector<char> host;
  for (auto& kv : pk->tensors) {
    const TensorMeta& m = kv.second;
    host.resize(m.nbytes);
    if (std::fseek(fp, static_cast<long>(m.offset), SEEK_SET) != 0 || std::fread(host.data(), 1, m.nbytes, fp) != m.nbytes)
      die("%s: tensor %s runs past the end of the file", path.c_str(), kv.first.c_str());
    void* d = nullptr;
    HIP_OK(hipMalloc(&d, m.nbytes));
    HIP_OK(hipMemcpy(d, host.data(), m.nbytes, hipMemcpyHostToDevice));
    pk->device_buffers.push_back(d);
    pk->dev[kv.first] = d;
  }
  std::fclose(fp);
}

void* need(Packed& pk, const std::string& name) {
  auto it = pk.dev.find(name);
  if (it == pk.dev.end()) die("weights file lacks tensor %s", name.c_str());
  return it->second;
}

// ------------------------------------------------------------------------------------------------
// Entry points: one graph-captured q4llm_step per (C, L)
// ------------------------------------------------------------------------------------------------

// Decode entry points (C == 1) feed themselves: their token buffer is their `next` buffer (q4llm_step
// reads the tokens in its first kernel and writes next in its last) and the step is q4llm_step_feed,
// whose last kernel adds 1 to start, so after a call the device inputs already hold what the
// following decode call passes; `call` then skips the host-to-device copy.
struct EntryPoint {
  int C = 0, L = 0;
  int32_t* io = nullptr;  // device allocation [C + 3] int32 holding the four buffers below
  int32_t *tokens = nullptr, *start = nullptr, *last = nullptr, *next = nullptr;  // device, inside io
  void* ws = nullptr;
  size_t ws_bytes = 0;
  hipGraphExec_t exec = nullptr;
  bool fed = false;  // decode only: the device holds (fed_start, fed_token, last = 0) as inputs
  int32_t fed_start = 0, fed_token = 0;
};

// K decode steps in one graph: step i reads the token in ring slot i - 1 (step 0: the last slot,
// the previous launch's last token) and writes its next token into slot i; every step is
// q4llm_step_feed, so a launch ends with start advanced by K and the inputs set for the next one.
struct DecodeRun {
  int L = 0, K = 0;
  int32_t* io = nullptr;  // device [K + 2]: ring[K], start, last
  int32_t *ring = nullptr, *start = nullptr, *last = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  hipGraphExec_t exec = nullptr;
  bool fed = false;
  int32_t fed_start = 0, fed_token = 0;
};

struct Runner {
  q4llm_model model{};
  std::vector<q4llm_layer> layers;
  std::vector<void*> caches;
  hipStream_t stream = nullptr;
  int32_t* host = nullptr;  // pinned: [0, C) tokens, then start, last, next
  int host_cap = 0;
  std::map<std::pair<int, int>, EntryPoint> eps;
  std::map<std::pair<int, int>, DecodeRun> runs;

  // decode entry points (feed) advance their own start in the step's last kernel
  void raw_step(EntryPoint& e, bool feed = false) {
    if (feed)
      Q4_OK_OR_DIE(q4llm_step_feed(&model, e.tokens, e.C, e.start, e.last, caches.data(), e.L, e.next, nullptr, e.ws,
                                   e.ws_bytes, stream));
    else
      Q4_OK_OR_DIE(q4llm_step(&model, e.tokens, e.C, e.start, e.last, caches.data(), e.L, e.next, nullptr, e.ws,
                              e.ws_bytes, stream));
  }

  EntryPoint& entry(int C, int L) {
    auto key = std::make_pair(C, L);
    auto it = eps.find(key);
    if (it != eps.end()) return it->second;
    EntryPoint e;
    e.C = C;
    e.L = L;
    HIP_OK(hipMalloc(&e.io, sizeof(int32_t) * (C + 3)));
    HIP_OK(hipMemset(e.io, 0, sizeof(int32_t) * (C + 3)));
    e.tokens = e.io;
    e.start = e.io + C;
    e.last = e.start + 1;
    e.next = e.last + 1;
    if (C == 1) e.tokens = e.next;
    Q4_OK_OR_DIE(q4llm_step_workspace_bytes(&model, C, L, &e.ws_bytes));
    HIP_OK(hipMalloc(&e.ws, e.ws_bytes));
    HIP_OK(hipMemset(e.ws, 0, e.ws_bytes));
    // First launch outside capture (code objects and LDS attributes are set up here), at position
    // max_ctx: the RoPE/KV-write kernels write no cache row there, so an entry point first built
    // after the prompt is in the caches (no warm-up) leaves that prompt's K/V rows intact.
    const int32_t setup_pos = model.max_ctx;
    HIP_OK(hipMemcpy(e.start, &setup_pos, sizeof(int32_t), hipMemcpyHostToDevice));
    raw_step(e);
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipMemset(e.io, 0, sizeof(int32_t) * (C + 3)));
    hipGraph_t g = nullptr;
    HIP_OK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    raw_step(e, C == 1);
    HIP_OK(hipStreamEndCapture(stream, &g));
    HIP_OK(hipGraphInstantiate(&e.exec, g, nullptr, nullptr, 0));
    HIP_OK(hipGraphDestroy(g));
    return eps.emplace(key, e).first->second;
  }

  DecodeRun& run_entry(int L, int K) {
    auto key = std::make_pair(L, K);
    auto it = runs.find(key);
    if (it != runs.end()) return it->second;
    DecodeRun d;
    d.L = L;
    d.K = K;
    HIP_OK(hipMalloc(&d.io, sizeof(int32_t) * (K + 2)));
    HIP_OK(hipMemset(d.io, 0, sizeof(int32_t) * (K + 2)));
    d.ring = d.io;
    d.start = d.io + K;
    d.last = d.start + 1;
    Q4_OK_OR_DIE(q4llm_step_workspace_bytes(&model, 1, L, &d.ws_bytes));
    HIP_OK(hipMalloc(&d.ws, d.ws_bytes));
    HIP_OK(hipMemset(d.ws, 0, d.ws_bytes));
    // set-up launch outside capture at position max_ctx (no cache row written), as in entry()
    const int32_t setup_pos = model.max_ctx;
    HIP_OK(hipMemcpy(d.start, &setup_pos, sizeof(int32_t), hipMemcpyHostToDevice));
    Q4_OK_OR_DIE(q4llm_step(&model, d.ring + K - 1, 1, d.start, d.last, caches.data(), L, d.ring, nullptr, d.ws,
                            d.ws_bytes, stream));
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipMemset(d.io, 0, sizeof(int32_t) * (K + 2)));
    hipGraph_t g = nullptr;
    HIP_OK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < K; ++i)
      Q4_OK_OR_DIE(q4llm_step_feed(&model, d.ring + (i + K - 1) % K, 1, d.start, d.last, caches.data(), L,
                                   d.ring + i, nullptr, d.ws, d.ws_bytes, stream));
    HIP_OK(hipStreamEndCapture(stream, &g));
    HIP_OK(hipGraphInstantiate(&d.exec, g, nullptr, nullptr, 0));
    HIP_OK(hipGraphDestroy(g));
    return runs.emplace(key, d).first->second;
  }

  // K decode steps from position start after token `token`: the K next tokens into out[0, K).
  void call_run(int L, int K, int32_t token, int start, int32_t* out) {
    DecodeRun& d = run_entry(L, K);
    if (K + 2 > host_cap) {
      if (host) HIP_OK(hipHostFree(host));
      host_cap = K + 2;
      HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&host), sizeof(int32_t) * host_cap, hipHostMallocDefault));
    }
    if (!(d.fed && d.fed_start == start && d.fed_token == token)) {
      host[0] = token;  // -> ring[K - 1]
      host[1] = start;
      host[2] = 0;  // last
      HIP_OK(hipMemcpyAsync(d.ring + K - 1, host, sizeof(int32_t) * 3, hipMemcpyHostToDevice, stream));
    }
    HIP_OK(hipGraphLaunch(d.exec, stream));
    HIP_OK(hipMemcpyAsync(host, d.ring, sizeof(int32_t) * K, hipMemcpyDeviceToHost, stream));
    HIP_OK(hipStreamSynchronize(stream));
    for (int i = 0; i < K; ++i) out[i] = host[i];
    d.fed = true;
    d.fed_start = start + K;
    d.fed_token = out[K - 1];
  }

  // One call of the entry point: token ids, start and last in, the greedy next token out.
  int32_t call(int C, int L, const int32_t* tokens, int n, int start, int last) {
    EntryPoint& e = entry(C, L);
    if (C + 3 > host_cap) {
      if (host) HIP_OK(hipHostFree(host));
      host_cap = C + 3;
      HIP_OK(hipHostMalloc(reinterpret_cast<void**>(&host), sizeof(int32_t) * host_cap, hipHostMallocDefault));
    }
    const bool fed = C == 1 && e.fed && e.fed_start == start && e.fed_token == tokens[0] && last == 0;
    if (!fed) {
      if (C == 1) {  // layout [start, last, next = tokens]
        host[0] = start;
        host[1] = last;
        host[2] = n > 0 ? tokens[0] : 0;
        HIP_OK(hipMemcpyAsync(e.start, host, sizeof(int32_t) * 3, hipMemcpyHostToDevice, stream));
      } else {
        for (int i = 0; i < C; ++i) host[i] = i < n ? tokens[i] : 0;
        host[C] = start;
        host[C + 1] = last;
        HIP_OK(hipMemcpyAsync(e.tokens, host, sizeof(int32_t) * (C + 2), hipMemcpyHostToDevice, stream));
      }
    }
    HIP_OK(hipGraphLaunch(e.exec, stream));
    HIP_OK(hipMemcpyAsync(host + C + 2, e.next, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    HIP_OK(hipStreamSynchronize(stream));
    const int32_t out = host[C + 2];
    if (C == 1) {
      e.fed = true;
      e.fed_start = start + 1;
      e.fed_token = out;
    }
    return out;
  }
};

void print_plan(const Plan& p) {
  std::printf("{\"prefill\":[");
  for (size_t i = 0; i < p.prefill.size(); ++i) std::printf("%s%d", i ? "," : "", p.prefill[i]);
  std::printf("],\"decode\":[");
  for (size_t i = 0; i < p.decode.size(); ++i) std::printf("%s%d", i ? "," : "", p.decode[i]);
  std::printf("]}\n");
}

}  // namespace

int main(int argc, char** argv) {
  const Flags f = parse_flags(argc, argv);
  if (f.prompt.empty()) die("--prompt is required");
  std::vector<int32_t> buckets = parse_ints(f.buckets);
  if (buckets.empty()) die("--buckets is empty");
  for (size_t i = 1; i < buckets.size(); ++i)
    if (buckets[i] <= buckets[i - 1]) die("--buckets must be ascending (%s)", f.buckets.c_str());
  const std::vector<int32_t> stops = parse_ints(f.stop_ids);
  const bool use_max = f.schedule == "max";
  const std::vector<int32_t> prompt = parse_ints(read_file(f.prompt));
  const int n_prompt = static_cast<int>(prompt.size());
  const int C = f.chunk;

  if (f.plan) {  // schedule only: no weights, no GPU
    const int max_ctx = f.max_ctx > 0 ? f.max_ctx : 4096;  // the reference flag default (llm_runner.c:42)
    print_plan(make_plan(n_prompt, f.max_new_tokens, C, buckets, max_ctx, use_max));
    return 0;
  }
  if (f.weights.empty()) die("--weights is required");

  Packed pk;
  load_packed(f.weights, &pk);
  auto cfg = [&](const char* k) { return static_cast<int>(pk.ints.at(k)); };
  auto agree = [&](int flag, const char* name, int value) {
    if (flag > 0 && flag != value) die("--%s=%d disagrees with the weights file (%d there)", name, flag, value);
  };
  agree(f.n_layers, "n_layers", cfg("n_layers"));
  agree(f.n_kv_heads, "n_kv_heads", cfg("n_kv"));
  agree(f.head_dim, "head_dim", cfg("head_dim"));
  agree(f.max_ctx, "max_ctx", cfg("max_ctx"));
  const Plan plan = make_plan(n_prompt, f.max_new_tokens, C, buckets, cfg("max_ctx"), use_max);
  if (buckets.back() > cfg("max_ctx")) die("bucket %d exceeds max_ctx %d", buckets.back(), cfg("max_ctx"));

  Runner r;
  const int nl = cfg("n_layers");
  r.layers.resize(nl);
  for (int i = 0; i < nl; ++i) {
    const std::string p = "layers." + std::to_string(i) + ".";
    q4llm_layer& ly = r.layers[i];
    ly.wqkv_q = static_cast<const int32_t*>(need(pk, p + "wqkv.qweight"));
    ly.wqkv_s = static_cast<const uint16_t*>(need(pk, p + "wqkv.scales"));
    ly.wo_q = static_cast<const int32_t*>(need(pk, p + "wo.qweight"));
    ly.wo_s = static_cast<const uint16_t*>(need(pk, p + "wo.scales"));
    ly.wgu_q = static_cast<const int32_t*>(need(pk, p + "wgu.qweight"));
    ly.wgu_s = static_cast<const uint16_t*>(need(pk, p + "wgu.scales"));
    ly.wdown_q = static_cast<const int32_t*>(need(pk, p + "wdown.qweight"));
    ly.wdown_s = static_cast<const uint16_t*>(need(pk, p + "wdown.scales"));
    ly.ln_in = static_cast<const float*>(need(pk, p + "ln_in"));
    ly.ln_post = static_cast<const float*>(need(pk, p + "ln_post"));
  }
  q4llm_model& m = r.model;
  m.dim = cfg("dim");
  m.n_layers = nl;
  m.n_heads = cfg("n_heads");
  m.n_kv = cfg("n_kv");
  m.head_dim = cfg("head_dim");
  m.inter = cfg("inter");
  m.vocab = cfg("vocab");
  m.group = cfg("group");
  m.max_ctx = cfg("max_ctx");
  m.eps = pk.eps;
  m.embed_q = static_cast<const int32_t*>(need(pk, "embed.qweight"));
  m.embed_s = static_cast<const uint16_t*>(need(pk, "embed.scales"));
  m.ln_f = static_cast<const float*>(need(pk, "ln_f"));
  m.cos_t = static_cast<const float*>(need(pk, "cos"));
  m.sin_t = static_cast<const float*>(need(pk, "sin"));
  m.layers = r.layers.data();

  // T16 copies of the decode projections and the LM head (q4_t16_pack), built on the device from the
  // reference layout; shapes the decode GEMV does not take keep none.
  auto t16 = [&](const int32_t* q, const uint16_t* sc, int64_t n, int64_t k, int pairing) {
    q4llm_t16 t{nullptr, nullptr};
    size_t tb = 0, sb = 0;
    const int st = q4_t16_bytes(n, k, m.group, pairing, m.head_dim, &tb, &sb);
    if (st == Q4_ERR_UNSUPPORTED) return t;
    Q4_OK_OR_DIE(st);
    void *tiles = nullptr, *tsc = nullptr;
    HIP_OK(hipMalloc(&tiles, tb));
    HIP_OK(hipMalloc(&tsc, sb));
    pk.device_buffers.push_back(tiles);
    pk.device_buffers.push_back(tsc);
    Q4_OK_OR_DIE(q4_t16_pack(q, sc, n, k, m.group, pairing, m.head_dim, tiles, tsc, nullptr));
    t.tiles = tiles;
    t.scales = tsc;
    return t;
  };
  const int64_t qkv_n = static_cast<int64_t>(m.n_heads + 2 * m.n_kv) * m.head_dim;
  for (auto& ly : r.layers) {
    ly.wqkv_t = t16(ly.wqkv_q, ly.wqkv_s, qkv_n, m.dim, Q4_PAIR_ROPE);
    ly.wo_t = t16(ly.wo_q, ly.wo_s, m.dim, static_cast<int64_t>(m.n_heads) * m.head_dim, Q4_PAIR_NONE);
    ly.wgu_t = t16(ly.wgu_q, ly.wgu_s, 2LL * m.inter, m.dim, Q4_PAIR_SWIGLU);
    ly.wdown_t = t16(ly.wdown_q, ly.wdown_s, m.dim, m.inter, Q4_PAIR_NONE);
  }
  m.embed_t = t16(m.embed_q, m.embed_s, m.vocab, m.dim, Q4_PAIR_NONE);
  HIP_OK(hipDeviceSynchronize());

  // KV caches: zeroed device buffers kept for the whole run (llm_runner.c:301-315).
  const size_t cache_bytes = static_cast<size_t>(m.max_ctx) * m.n_kv * m.head_dim * 2;
  r.caches.resize(2 * nl);
  for (auto& c : r.caches) {
    HIP_OK(hipMalloc(&c, cache_bytes));
    HIP_OK(hipMemset(c, 0, cache_bytes));
  }
  HIP_OK(hipStreamCreate(&r.stream));

  // Warm-up of every entry point the schedule uses (graph capture included), outside the timings.
  // The calls write garbage KV at [0, C) that prefill overwrites before anything reads it.
  const std::vector<int32_t> zeros(C, 0);
  const double tw = now_ms();
  std::vector<int> used_pre(plan.prefill), used_dec(plan.decode);
  for (int w = 0; w < f.warmup; ++w) {
    for (int L : buckets) {
      for (int u : used_pre)
        if (u == L) {
          r.call(C, L, zeros.data(), C, 0, 0);
          break;
        }
      for (int u : used_dec)
        if (u == L) {
          r.call(1, L, zeros.data(), 1, 0, 0);
          break;
        }
      // the K-step graph of a bucket that holds K decode steps: built (captured), not run
      if (f.decode_steps > 1 && std::count(used_dec.begin(), used_dec.end(), L) >= f.decode_steps)
        r.run_entry(L, f.decode_steps);
    }
  }
  const double warm_ms = now_ms() - tw;

  // Prefill (chunked, last chunk zero padded).
  std::vector<std::pair<int, double>> chunks, steps;
  std::vector<int32_t> generated;
  int32_t next = 0;
  const double t0 = now_ms();
  for (int start = 0, i = 0; start < n_prompt; start += C, ++i) {
    const int n = std::min(C, n_prompt - start);
    const double tc = now_ms();
    next = r.call(C, plan.prefill[i], prompt.data() + start, n, start, n - 1);
    chunks.emplace_back(plan.prefill[i], now_ms() - tc);
  }
  const double prefill_ms = now_ms() - t0;

  // Decode: the first token comes from prefill.
  generated.push_back(next);
  const double t1 = now_ms();
  int pos = n_prompt;
  while (static_cast<int>(generated.size()) < f.max_new_tokens) {
    bool stop = false;
    for (int s : stops) stop = stop || next == s;
    if (stop) break;
    const int L = pick_bucket(buckets, pos + 1, use_max);
    if (L < 0) break;
    const int K = f.decode_steps;
    const bool run = K > 1 && static_cast<int>(generated.size()) + K <= f.max_new_tokens &&
                     pick_bucket(buckets, pos + K, use_max) == L;
    const double ts = now_ms();
    const int32_t tok = next;
    if (!run) {
      next = r.call(1, L, &tok, 1, pos, 0);
      steps.emplace_back(L, now_ms() - ts);
      generated.push_back(next);
      ++pos;
      continue;
    }
    std::vector<int32_t> outs(K);
    r.call_run(L, K, tok, pos, outs.data());
    const double per = (now_ms() - ts) / K;
    for (int i = 0; i < K; ++i) {
      next = outs[i];
      steps.emplace_back(L, per);
      generated.push_back(next);
      ++pos;
      bool hit = false;
      for (int s : stops) hit = hit || next == s;
      if (hit) break;
    }
  }
  const double decode_ms = now_ms() - t1;
  const int n_steps = static_cast<int>(generated.size()) - 1;

  std::printf("{\"schedule\":\"%s\",\"chunk\":%d,\"prompt_tokens\":%d,\"new_tokens\":%d,", f.schedule.c_str(), C,
              n_prompt, static_cast<int>(generated.size()));
  std::printf("\"warmup_ms\":%.1f,\"prefill_ms\":%.1f,\"prefill_tok_s\":%.2f,\"ttft_ms\":%.1f,", warm_ms, prefill_ms,
              n_prompt / (prefill_ms / 1e3), prefill_ms);
  std::printf("\"decode_ms\":%.1f,\"decode_steps\":%d,\"decode_tok_s\":%.2f,", decode_ms, n_steps,
              n_steps > 0 ? n_steps / (decode_ms / 1e3) : 0.0);
  std::printf("\"chunks\":[");
  for (size_t i = 0; i < chunks.size(); ++i) std::printf("%s[%d,%.1f]", i ? "," : "", chunks[i].first, chunks[i].second);
  std::printf("],\"steps\":[");
  for (size_t i = 0; i < steps.size(); ++i) std::printf("%s[%d,%.2f]", i ? "," : "", steps[i].first, steps[i].second);
  std::printf("],\"tokens\":[");
  for (size_t i = 0; i < generated.size(); ++i) std::printf("%s%d", i ? "," : "", generated[i]);
  std::printf("]}\n");
  std::fflush(stdout);

  for (auto& kv : r.eps) {
    HIP_OK(hipGraphExecDestroy(kv.second.exec));
    HIP_OK(hipFree(kv.second.ws));
    HIP_OK(hipFree(kv.second.io));
  }
  for (auto& kv : r.runs) {
    HIP_OK(hipGraphExecDestroy(kv.second.exec));
    HIP_OK(hipFree(kv.second.ws));
    HIP_OK(hipFree(kv.second.io));
  }
  for (void* c : r.caches) HIP_OK(hipFree(c));
  for (void* d : pk.device_buffers) HIP_OK(hipFree(d));
  if (r.host) HIP_OK(hipHostFree(r.host));
  HIP_OK(hipStreamDestroy(r.stream));
  return 0;
}
