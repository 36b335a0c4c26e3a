// Native BitNet engine behind the reference's engine C ABI (include/wfbitnet_engine.h), built on the
// libwfbitnet entry points.
//
// The reference runs one token at a time on the CPU, prompt included
// (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:490-554, 742-823).  Here:
//  * the weights, the KV cache and every work buffer live in HBM from bitnet_engine_create on;
//    q|k|v and gate|up are concatenated at load time into one segmented weight each;
//  * the float glue (embedding, norms, residual stream, KV cache, attention, dense LM head) is fp32 for a
//    file whose config says torch_dtype float32 (or, without that key, stores its embedding in float32), as
//    the reference engine computes; otherwise bf16 (half the bytes of the residual stream, the cache and a
//    dense head);
//  * a prompt is one batched pass: the layer sequence at M = prompt length (prefill GEMMs; bf16: matrix-core
//    prefill attention with the cache append, fp32: one decode attention per position), its last row kept as
//    the pending hidden state;
//  * a generated token is one replay of a HIP graph captured once per engine:
//      LM head (final RMSNorm + head + first-max argmax)  -> token on the device
//      embedding row of that token -> the layer sequence at M = 1 (decode attention at the device
//      position) -> commit (token recorded, hidden state kept in a small ring, position + 1);
//    greedy generation replays it in chunks of kChunk with one host synchronisation per chunk;
//  * sampling (temperature > 0) replays the head alone with the logits stored, samples on the host
//    with the reference's algorithm (bitnet_engine.cpp:208-253, 782-788) and replays the rest.
// Every layer step issues exactly the calls the Python model's fused HIP backend issues for the same
// rows (wrinklefree-monorepo_amd/model.py, HipBackend(fused=True) with bf16 glue, or fp32 glue with
// prefill_attention="steps"), so both produce the same tokens bit for bit.  This file is host code only; the engine's own small kernels (embedding rows,
// float conversion at load, the decode step's commit, the hidden-state restore) are in engine_kernels.hip.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <utility>
#include <vector>

#include "../../include/wfbitnet_engine.h"
#include "engine_kernels.h"
#include "wfb_common.h"

namespace {

thread_local std::string g_eng_err;

int efail(const std::string& msg) {
  g_eng_err = msg;
  return -1;
}

// ---- SGLBITNT file (format of SGB/sgl-kernel/csrc/inference/sglkernel_loader.h:1-20) -------------

struct TensorRec {
  uint32_t dtype = 0;  // 0 uint8, 1 float32, 2 float16, 3 bfloat16
  std::vector<int64_t> shape;
  bool has_scale = false;
  float scale = 1.0f;
  size_t offset = 0, nbytes = 0;
  // element count, or -1 when it does not fit in 62 bits (a corrupt header)
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape)
      if (__builtin_mul_overflow(n, d, &n) || n > ((int64_t)1 << 62)) return -1;
    return n;
  }
};

struct ModelFile {
  int fd = -1;
  const uint8_t* base = nullptr;
  size_t size = 0;
  std::string json;
  std::vector<std::pair<std::string, TensorRec>> tensors;
  ~ModelFile() {
    if (base) munmap(const_cast<uint8_t*>(base), size);
    if (fd >= 0) close(fd);
  }
  const TensorRec* find(const std::string& name) const {
    for (const auto& t : tensors)
      if (t.first == name) return &t.second;
    return nullptr;
  }
};

int open_model(const char* path, ModelFile& f) {
  if (!path) return efail("Failed to open file: (null)");
  f.fd = open(path, O_RDONLY);
  if (f.fd < 0) return efail(std::string("Failed to open file: ") + path);
  struct stat st;
  if (fstat(f.fd, &st) != 0 || st.st_size < 16) return efail(std::string("Failed to read file: ") + path);
  f.size = (size_t)st.st_size;
  void* p = mmap(nullptr, f.size, PROT_READ, MAP_PRIVATE, f.fd, 0);
  if (p == MAP_FAILED) return efail(std::string("Failed to map file: ") + path);
  f.base = static_cast<const uint8_t*>(p);
  size_t at = 0;
  auto take = [&](void* dst, size_t n) -> bool {
    if (n > f.size - at) return false;
    std::memcpy(dst, f.base + at, n);
    at += n;
    return true;
  };
  char magic[8];
  uint32_t version = 0, clen = 0, count = 0;
  if (!take(magic, 8) || std::memcmp(magic, "SGLBITNT", 8) != 0) return efail("Invalid magic number");
  if (!take(&version, 4)) return efail("Truncated file");
  if (version != 1) return efail("Unsupported version: " + std::to_string(version));
  if (!take(&clen, 4) || clen > f.size - at) return efail("Truncated config");
  f.json.assign(reinterpret_cast<const char*>(f.base + at), clen);
  at += clen;
  if (!take(&count, 4)) return efail("Truncated tensor table");
  for (uint32_t i = 0; i < count; ++i) {
    uint32_t nlen = 0, ndims = 0, has_scale = 0;
    uint64_t nbytes = 0;
    if (!take(&nlen, 4) || nlen > f.size - at) return efail("Truncated tensor table");
    std::string name(reinterpret_cast<const char*>(f.base + at), nlen);
    at += nlen;
    TensorRec t;
    if (!take(&t.dtype, 4) || !take(&ndims, 4) || ndims > 8) return efail("Bad tensor header: " + name);
    if (t.dtype > 3) return efail("Unknown dtype id " + std::to_string(t.dtype) + " of " + name);
    for (uint32_t d = 0; d < ndims; ++d) {
      uint32_t v = 0;
      if (!take(&v, 4)) return efail("Bad tensor header: " + name);
      t.shape.push_back((int64_t)v);
    }
    if (!take(&has_scale, 4)) return efail("Bad tensor header: " + name);
    t.has_scale = has_scale == 1;
    if (t.has_scale && !take(&t.scale, 4)) return efail("Bad tensor header: " + name);
    if (!take(&nbytes, 8) || nbytes > f.size - at) return efail("Truncated tensor data: " + name);
    const int64_t esize = t.dtype == 0 ? 1 : t.dtype == 1 ? 4 : 2;
    if (t.numel() < 0 || (uint64_t)(t.numel() * esize) != nbytes)
      return efail("Tensor size does not match its shape: " + name);
    t.offset = at;
    t.nbytes = nbytes;
    at += nbytes;
    f.tensors.emplace_back(std::move(name), std::move(t));
  }
  return 0;
}

// The value text after "key": in a JSON object (first occurrence, as the reference's parse_config);
// empty when absent.
std::string json_raw(const std::string& js, const char* key) {
  const std::string k = std::string("\"") + key + "\"";
  size_t p = js.find(k);
  if (p == std::string::npos) return "";
  p = js.find(':', p + k.size());
  if (p == std::string::npos) return "";
  ++p;
  while (p < js.size() && (js[p] == ' ' || js[p] == '\t' || js[p] == '\n' || js[p] == '\r')) ++p;
  size_t e = p;
  if (e < js.size() && js[e] == '"') {
    e = js.find('"', p + 1);
    return e == std::string::npos ? "" : js.substr(p, e - p + 1);
  }
  if (e < js.size() && js[e] == '[') {
    e = js.find(']', p);
    return e == std::string::npos ? "" : js.substr(p, e - p + 1);
  }
  while (e < js.size() && js[e] != ',' && js[e] != '}' && js[e] != '\n') ++e;
  std::string v = js.substr(p, e - p);
  while (!v.empty() && (v.back() == ' ' || v.back() == '\r' || v.back() == '\t')) v.pop_back();
  return v;
}

bool json_num(const std::string& js, const char* key, double& out) {
  const std::string v = json_raw(js, key);
  if (v.empty() || v == "null") return false;
  char* end = nullptr;
  const double d = std::strtod(v.c_str(), &end);
  if (end == v.c_str()) return false;
  out = d;
  return true;
}

// ---- the engine ---------------------------------------------------------------------------------

constexpr int kChunk = 32;          // greedy decode steps replayed between host synchronisations
constexpr int kRing = kChunk + 1;   // hidden states kept (restores the state at an EOS inside a chunk)

struct Cfg {
  int64_t vocab = 0, hidden = 0, inter = 0, layers = 0, heads = 0, kv_heads = 0, head_dim = 0, max_len = 0;
  double theta = 10000.0;
  float rms_eps = 1e-5f, subln_eps = 1e-6f;
  int act = WFB_ACT_SILU;
  std::vector<int64_t> eos;
  int64_t qd() const { return heads * head_dim; }
  int64_t kvd() const { return kv_heads * head_dim; }
  int64_t nqkv() const { return qd() + 2 * kvd(); }
};

struct Layer {
  uint8_t *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;
  float* scales = nullptr;  // device [7]: q, k, v, o, gate, up, down
  // float vectors in the engine's glue dtype (bf16 or fp32, Engine::gdt)
  void *in_norm = nullptr, *post_norm = nullptr, *attn_sub = nullptr, *ffn_sub = nullptr;
  void *kc = nullptr, *vc = nullptr;  // [kv_heads, max_len, head_dim]
};

// Work buffers of one row count (the decode set holds 1 row, the prompt set grows with the prompt).
struct Acts {
  int64_t cap = 0;
  void* x = nullptr;         // [cap, H] residual stream (glue dtype)
  void* qkv = nullptr;       // [cap, Nqkv] (glue dtype)
  void* att = nullptr;       // [cap, qd] (glue dtype)
  int8_t* codes = nullptr;   // [cap, kmax]
  float* ascale = nullptr;   // [cap]
  float* mid = nullptr;      // [min(cap, 64), F] gated product of the M <= 64 path
  void* gu = nullptr;        // [cap, 2F] gate|up outputs (glue dtype) of the M > 64 path (and of every M when F % 32 != 0)
  int64_t* ids = nullptr;    // [cap] token ids of the embedding gather
};

}  // namespace

struct BitNetEngine {
  Cfg c;
  int device = 0;
  hipStream_t s = nullptr;
  std::vector<void*> allocs;  // every device allocation, freed at destroy
  int64_t kpad_h = 0, kpad_qd = 0, kpad_f = 0, kmax = 0;
  int64_t seg_qkv[3] = {0, 0, 0};
  // Glue dtype: WFB_BF16, or WFB_F32 for a file whose config says torch_dtype float32 (or, without that key,
  // whose embedding is stored in float32) -- the reference engine's arithmetic (bitnet_engine.cpp:107,
  // 146-150, 289, 541-553): embedding, norms, residual stream, KV cache, attention and a dense head in fp32.
  int gdt = WFB_BF16;
  int64_t es = 2;                 // its element size
  int64_t* iota = nullptr;        // device [max_len] = 0, 1, ... (fp32 prompts: one decode attention per position)
  void* embed = nullptr;
  std::vector<Layer> L;
  void* final_norm = nullptr;
  uint8_t* head_q = nullptr;      // ternary head [V, kpad_h/4]
  float* head_scale = nullptr;    // device [1]
  void* head_dense = nullptr;     // dense head [V, H] (the embedding when tied)
  float *rope_cos = nullptr, *rope_sin = nullptr;
  Acts dec, pre;
  float* attn_ws = nullptr;
  uint64_t* argmax_ws = nullptr;
  int64_t* ctl = nullptr;          // device {token, position, count}
  int64_t* ctl_h = nullptr;        // pinned host mirror
  int32_t* tokens = nullptr;       // device [max_len] tokens of a greedy generation
  int32_t* last_tok = nullptr;     // device [1]
  void* ring = nullptr;            // device [kRing, H]
  void* x_start = nullptr;         // device [H] hidden state before the first generated token
  void* logits = nullptr;          // device [V] fp32
  void* logits_h = nullptr;        // pinned host copy
  int64_t* ids_h = nullptr;        // pinned host prompt ids (pre.cap)
  int32_t* tokens_h = nullptr;     // pinned host [kChunk]
  hipGraphExec_t g_greedy = nullptr, g_head = nullptr, g_body = nullptr;
  std::mt19937 rng{42};
  int64_t seq_len = 0;
  bool have_hidden = false;

  ~BitNetEngine() {
    if (s) (void)hipStreamSynchronize(s);
    for (hipGraphExec_t g : {g_greedy, g_head, g_body})
      if (g) (void)hipGraphExecDestroy(g);
    for (void* p : allocs) (void)hipFree(p);
    for (void* p : {(void*)ctl_h, logits_h, (void*)ids_h, (void*)tokens_h})
      if (p) (void)hipHostFree(p);
    if (s) (void)hipStreamDestroy(s);
  }
};

namespace {

using Engine = BitNetEngine;

int hipfail(hipError_t e, const char* what) {
  return efail(std::string(what) + ": HIP error " + std::to_string((int)e) + " (" + hipGetErrorString(e) + ")");
}

// A libwfbitnet status to the engine's error channel.
int wcheck(int st, const char* what) {
  if (st == WFB_OK) return 0;
  return efail(std::string(what) + ": " + wfb_last_error());
}

#define ECHECK(x)                  \
  do {                             \
    const int st_ = (x);           \
    if (st_ != 0) return st_;      \
  } while (0)
#define HCHECK(x, what)                         \
  do {                                          \
    const hipError_t e_ = (x);                  \
    if (e_ != hipSuccess) return hipfail(e_, what); \
  } while (0)

// Allocations left before the engine's allocator reports a failure; negative = never (the default).
// Set only through wfb_engine_fail_alloc_after, which tests use to reach the out-of-memory paths.
std::atomic<int64_t> g_fail_alloc_after{-1};

int alloc_gate(const char* what) {
  int64_t n = g_fail_alloc_after.load();
  while (n > 0 && !g_fail_alloc_after.compare_exchange_weak(n, n - 1)) {
  }
  if (n == 0) return efail(std::string(what) + ": allocation failure injected (wfb_engine_fail_alloc_after)");
  return 0;
}

template <typename T>
int dalloc(Engine& e, T*& p, size_t count) {
  ECHECK(alloc_gate("hipMalloc"));
  void* q = nullptr;
  const hipError_t st = hipMalloc(&q, std::max<size_t>(count * sizeof(T), 256));
  if (st != hipSuccess) return hipfail(st, "hipMalloc");
  e.allocs.push_back(q);
  p = static_cast<T*>(q);
  return 0;
}

int dalloc_bytes(Engine& e, void*& p, size_t bytes) {
  uint8_t* q = nullptr;
  ECHECK(dalloc(e, q, bytes));
  p = q;
  return 0;
}

void dfree(Engine& e, void* p) {
  if (!p) return;
  (void)hipFree(p);
  e.allocs.erase(std::remove(e.allocs.begin(), e.allocs.end(), p), e.allocs.end());
}

// n elements of the glue dtype
int galloc(Engine& e, void*& p, int64_t n) { return dalloc_bytes(e, p, (size_t)n * (size_t)e.es); }

// element i of a glue-dtype buffer
void* at(const Engine& e, void* p, int64_t i) { return static_cast<char*>(p) + i * e.es; }
const void* at(const Engine& e, const void* p, int64_t i) { return static_cast<const char*>(p) + i * e.es; }

int check_packed(const ModelFile& f, const std::string& name, int64_t out_rows, int64_t in_features) {
  const TensorRec* t = f.find(name);
  if (!t) return efail("Tensor not found: " + name);
  if (t->dtype != 0 || t->shape.size() != 2) return efail(name + ": expected a packed uint8 [out, in/4] weight");
  const int64_t kpad = t->shape[1] * 4;
  if (t->shape[0] != out_rows || kpad % WFB_QK_I2S != 0 || kpad < in_features || kpad >= in_features + WFB_QK_I2S)
    return efail(name + ": packed shape [" + std::to_string(t->shape[0]) + ", " + std::to_string(t->shape[1]) +
                 "] does not fit " + std::to_string(out_rows) + " x " + std::to_string(in_features));
  return 0;
}

int check_floats(const ModelFile& f, const std::string& name, int64_t numel, bool optional) {
  const TensorRec* t = f.find(name);
  if (!t) return optional ? 0 : efail("Tensor not found: " + name);
  if (t->dtype == 0) return efail(name + ": expected a float tensor");
  if (t->numel() != numel)
    return efail(name + ": " + std::to_string(t->numel()) + " elements, expected " + std::to_string(numel));
  return 0;
}

// Every tensor the model needs, with its dtype and shape (bitnet_engine.cpp:595-673 reads the same names).
int check_tensors(const ModelFile& f, const Cfg& c) {
  const int64_t H = c.hidden, F = c.inter, qd = c.qd(), kvd = c.kvd(), V = c.vocab;
  ECHECK(check_floats(f, "model.embed_tokens.weight", V * H, false));
  for (int64_t i = 0; i < c.layers; ++i) {
    const std::string pre = "model.layers." + std::to_string(i) + ".";
    ECHECK(check_packed(f, pre + "self_attn.q_proj.weight", qd, H));
    ECHECK(check_packed(f, pre + "self_attn.k_proj.weight", kvd, H));
    ECHECK(check_packed(f, pre + "self_attn.v_proj.weight", kvd, H));
    ECHECK(check_packed(f, pre + "self_attn.o_proj.weight", H, qd));
    ECHECK(check_packed(f, pre + "mlp.gate_proj.weight", F, H));
    ECHECK(check_packed(f, pre + "mlp.up_proj.weight", F, H));
    ECHECK(check_packed(f, pre + "mlp.down_proj.weight", H, F));
    ECHECK(check_floats(f, pre + "input_layernorm.weight", H, false));
    ECHECK(check_floats(f, pre + "post_attention_layernorm.weight", H, false));
    ECHECK(check_floats(f, pre + "self_attn.attn_sub_norm.weight", qd, true));
    ECHECK(check_floats(f, pre + "mlp.ffn_sub_norm.weight", F, true));
  }
  ECHECK(check_floats(f, "model.norm.weight", H, false));
  if (const TensorRec* t = f.find("lm_head.weight")) {
    if (t->dtype == 0) return check_packed(f, "lm_head.weight", V, H);
    return check_floats(f, "lm_head.weight", V * H, false);
  }
  return 0;
}

// Host bytes -> device, through a pinned staging buffer.
struct Uploader {
  Engine& e;
  void* stage = nullptr;
  size_t cap = 64u << 20;
  explicit Uploader(Engine& en) : e(en) {}
  ~Uploader() {
    if (stage) {
      (void)hipStreamSynchronize(e.s);
      (void)hipHostFree(stage);
    }
  }
  int put(void* dst, const uint8_t* src, size_t n) {
    if (!stage) HCHECK(hipHostMalloc(&stage, cap, hipHostMallocDefault), "hipHostMalloc");
    for (size_t off = 0; off < n; off += cap) {
      const size_t len = std::min(cap, n - off);
      HCHECK(hipStreamSynchronize(e.s), "upload");
      std::memcpy(stage, src + off, len);
      HCHECK(hipMemcpyAsync(static_cast<uint8_t*>(dst) + off, stage, len, hipMemcpyHostToDevice, e.s), "upload");
    }
    return 0;
  }
};

int load_packed(Uploader& up, const ModelFile& f, const std::string& name, int64_t out_rows, int64_t in_features,
                uint8_t* dst, std::vector<float>& scales_h, int slot) {
  ECHECK(check_packed(f, name, out_rows, in_features));
  const TensorRec* t = f.find(name);
  ECHECK(up.put(dst, f.base + t->offset, t->nbytes));
  scales_h[slot] = t->has_scale ? t->scale : 1.0f;
  return 0;
}

// A float tensor of `numel` elements in the glue dtype on the device; absent (optional) -> ones.
int load_floats(Engine& e, Uploader& up, const ModelFile& f, const std::string& name, int64_t numel, void* dst,
                bool optional, void* scratch, size_t scratch_bytes) {
  const TensorRec* t = f.find(name);
  if (!t) {
    if (!optional) return efail("Tensor not found: " + name);
    if (e.gdt == WFB_F32) {
      std::vector<float> ones((size_t)numel, 1.0f);
      return up.put(dst, reinterpret_cast<const uint8_t*>(ones.data()), (size_t)numel * 4);
    }
    std::vector<uint16_t> ones((size_t)numel, 0x3F80);
    return up.put(dst, reinterpret_cast<const uint8_t*>(ones.data()), (size_t)numel * 2);
  }
  if (t->dtype == 0) return efail(name + ": expected a float tensor");
  if (t->numel() != numel)
    return efail(name + ": " + std::to_string(t->numel()) + " elements, expected " + std::to_string(numel));
  const int64_t esize = t->dtype == 1 ? 4 : 2;
  const int64_t per = (int64_t)(scratch_bytes / esize);
  for (int64_t off = 0; off < numel; off += per) {
    const int64_t len = std::min(per, numel - off);
    ECHECK(up.put(scratch, f.base + t->offset + off * esize, (size_t)(len * esize)));
    HCHECK(wfb::launch_to_float(scratch, (int)t->dtype, len, at(e, dst, off), e.gdt, e.s), "float conversion");
  }
  return 0;
}

void free_acts(Engine& e, Acts& a) {
  for (void* p : {(void*)a.x, (void*)a.qkv, (void*)a.att, (void*)a.codes, (void*)a.ascale, (void*)a.mid, (void*)a.gu,
                  (void*)a.ids})
    dfree(e, p);
  a = Acts{};
}

// All buffers of `a` for `cap` rows; on failure the ones already made are freed and `a` is left empty
// (cap 0), so the next call that needs them allocates again.
int alloc_acts(Engine& e, Acts& a, int64_t cap) {
  const Cfg& c = e.c;
  Acts n;
  int st = galloc(e, n.x, cap * c.hidden);
  if (st == 0) st = galloc(e, n.qkv, cap * c.nqkv());
  if (st == 0) st = galloc(e, n.att, cap * c.qd());
  if (st == 0) st = dalloc(e, n.codes, cap * e.kmax);
  if (st == 0) st = dalloc(e, n.ascale, cap);
  if (st == 0) st = dalloc(e, n.mid, std::min<int64_t>(cap, 64) * c.inter);
  if (st == 0 && (cap > 64 || c.inter % 32 != 0)) st = galloc(e, n.gu, cap * 2 * c.inter);
  if (st == 0) st = dalloc(e, n.ids, cap);
  if (st != 0) {
    free_acts(e, n);
    a = Acts{};
    return st;
  }
  n.cap = cap;
  a = n;
  return 0;
}

// The fused norm + linear launches take these sizes (the Python backend's rmsnorm_linear_supported and
// rmsnorm_linear_glu_supported): up to 16 rows of up to 4096 elements; the plain linear also one row of
// 4097 .. 16384 elements.
bool fused_glu_ok(int64_t m, int64_t h, int64_t k) {
  return m >= 1 && m <= 16 && h % 8 == 0 && h > 0 && h <= k && k <= 4096 && k % WFB_QK_I2S == 0;
}
bool fused_norm_ok(int64_t m, int64_t h, int64_t k) {
  if (h % 8 != 0 || h <= 0 || h > k || k % WFB_QK_I2S != 0) return false;
  return (m >= 1 && m <= 16 && k <= 4096) || (m == 1 && k <= WFB_NORM_MAX_H);
}

// residual + linear(quantise(norm(x))) into the residual stream x (in place), one projection.
int norm_linear_residual(Engine& e, Acts& a, int64_t m, const void* x, int xdt, int64_t h, const void* gamma,
                         float eps, const uint8_t* w, int64_t kpad, const float* scale) {
  const Cfg& c = e.c;
  void* st = e.s;
  const int g = e.gdt;
  if (fused_norm_ok(m, h, kpad)) {
    const int64_t rows = c.hidden;
    return wcheck(wfb_rmsnorm_linear_i2s(x, xdt, h, gamma, g, eps, m, h, w, c.hidden, kpad, 1, &rows, scale, a.x, g,
                                         c.hidden, a.x, g, c.hidden, st),
                  "rmsnorm_linear (residual)");
  }
  ECHECK(wcheck(wfb_rmsnorm_quant_i8(x, xdt, h, gamma, g, eps, m, h, a.codes, kpad, kpad, a.ascale, st),
                "rmsnorm_quant"));
  return wcheck(wfb_linear_i2s_residual(w, c.hidden, kpad, a.codes, m, kpad, a.ascale, scale, 0.0f, a.x, g, c.hidden,
                                        a.x, g, c.hidden, st),
                "linear_residual");
}

// One decoder layer over the m rows of a.x.  prompt: rows are positions 0..m-1 (prefill attention; in fp32,
// which the matrix-core prefill kernel does not take, one decode attention per position, as the reference
// engine runs every prompt token through its attention, bitnet_engine.cpp:381-441); else one row at the device
// position ctl[1] (decode attention).
int layer(Engine& e, const Layer& Ly, Acts& a, int64_t m, bool prompt) {
  const Cfg& c = e.c;
  void* st = e.s;
  const int g = e.gdt;
  const int64_t H = c.hidden, F = c.inter, qd = c.qd(), kvd = c.kvd(), nqkv = c.nqkv();
  const float scale = (float)(1.0 / std::sqrt((double)c.head_dim));
  // RMSNorm -> q|k|v
  if (fused_norm_ok(m, H, e.kpad_h)) {
    ECHECK(wcheck(wfb_rmsnorm_linear_i2s(a.x, g, H, Ly.in_norm, g, c.rms_eps, m, H, Ly.qkv, nqkv, e.kpad_h, 3,
                                         e.seg_qkv, Ly.scales, nullptr, WFB_F32, nqkv, a.qkv, g, nqkv, st),
                  "rmsnorm_linear (q|k|v)"));
  } else {
    ECHECK(wcheck(wfb_rmsnorm_quant_i8(a.x, g, H, Ly.in_norm, g, c.rms_eps, m, H, a.codes, e.kpad_h, e.kpad_h,
                                       a.ascale, st),
                  "rmsnorm_quant"));
    ECHECK(wcheck(wfb_linear_i2s_segmented(Ly.qkv, nqkv, e.kpad_h, 3, e.seg_qkv, Ly.scales, a.codes, m, e.kpad_h,
                                           a.ascale, nullptr, WFB_F32, a.qkv, g, nqkv, nullptr, st),
                  "linear_segmented (q|k|v)"));
  }
  // rotary embedding + cache append + attention
  if (prompt && g == WFB_BF16) {
    ECHECK(wcheck(wfb_gqa_prefill_attention(a.qkv, nqkv, at(e, a.qkv, qd), nqkv, at(e, a.qkv, qd + kvd), nqkv, g,
                                            e.rope_cos, e.rope_sin, Ly.kc, Ly.vc, c.max_len, 0, 1, m, c.heads,
                                            c.kv_heads, c.head_dim, scale, a.att, qd, st),
                  "prefill attention"));
  } else if (prompt) {
    for (int64_t i = 0; i < m; ++i) {
      const int64_t r = i * nqkv;
      ECHECK(wcheck(wfb_gqa_decode_attention(at(e, a.qkv, r), nqkv, at(e, a.qkv, r + qd), nqkv,
                                             at(e, a.qkv, r + qd + kvd), nqkv, g, e.rope_cos, e.rope_sin, Ly.kc, Ly.vc,
                                             c.max_len, e.iota + i, 1, c.heads, c.kv_heads, c.head_dim, scale,
                                             at(e, a.att, i * qd), qd, e.attn_ws, st),
                    "decode attention (prompt)"));
    }
  } else {
    ECHECK(wcheck(wfb_gqa_decode_attention(a.qkv, nqkv, at(e, a.qkv, qd), nqkv, at(e, a.qkv, qd + kvd), nqkv, g,
                                           e.rope_cos, e.rope_sin, Ly.kc, Ly.vc, c.max_len, e.ctl + 1, 1, c.heads,
                                           c.kv_heads, c.head_dim, scale, a.att, qd, e.attn_ws, st),
                  "decode attention"));
  }
  // SubLN -> o + residual
  ECHECK(norm_linear_residual(e, a, m, a.att, g, qd, Ly.attn_sub, c.subln_eps, Ly.o, e.kpad_qd, Ly.scales + 3));
  // RMSNorm -> gate|up -> act(gate) * up -> SubLN -> down + residual
  if (m <= 64 && F % 32 == 0) {
    if (fused_glu_ok(m, H, e.kpad_h)) {
      ECHECK(wcheck(wfb_rmsnorm_linear_i2s_glu(a.x, g, H, Ly.post_norm, g, c.rms_eps, m, H, Ly.gu, 2 * F, e.kpad_h,
                                               Ly.scales + 4, c.act, g, a.mid, F, st),
                    "rmsnorm_linear_glu"));
    } else {
      ECHECK(wcheck(wfb_rmsnorm_quant_i8(a.x, g, H, Ly.post_norm, g, c.rms_eps, m, H, a.codes, e.kpad_h, e.kpad_h,
                                         a.ascale, st),
                    "rmsnorm_quant"));
      ECHECK(wcheck(wfb_linear_i2s_glu(Ly.gu, 2 * F, e.kpad_h, a.codes, m, e.kpad_h, a.ascale, Ly.scales + 4, c.act, g,
                                       a.mid, F, st),
                    "linear_glu"));
    }
    return norm_linear_residual(e, a, m, a.mid, WFB_F32, F, Ly.ffn_sub, c.subln_eps, Ly.down, e.kpad_f, Ly.scales + 6);
  }
  const int64_t seg_gu[2] = {F, F};
  if (fused_norm_ok(m, H, e.kpad_h)) {
    ECHECK(wcheck(wfb_rmsnorm_linear_i2s(a.x, g, H, Ly.post_norm, g, c.rms_eps, m, H, Ly.gu, 2 * F, e.kpad_h, 2, seg_gu,
                                         Ly.scales + 4, nullptr, WFB_F32, 2 * F, a.gu, g, 2 * F, st),
                  "rmsnorm_linear (gate|up)"));
  } else {
    ECHECK(wcheck(wfb_rmsnorm_quant_i8(a.x, g, H, Ly.post_norm, g, c.rms_eps, m, H, a.codes, e.kpad_h, e.kpad_h,
                                       a.ascale, st),
                  "rmsnorm_quant"));
    ECHECK(wcheck(wfb_linear_i2s_segmented(Ly.gu, 2 * F, e.kpad_h, 2, seg_gu, Ly.scales + 4, a.codes, m, e.kpad_h,
                                           a.ascale, nullptr, WFB_F32, a.gu, g, 2 * F, nullptr, st),
                  "linear_segmented (gate|up)"));
  }
  ECHECK(wcheck(wfb_glu_rmsnorm_quant_i8(a.gu, at(e, a.gu, F), g, 2 * F, c.act, Ly.ffn_sub, g, c.subln_eps, m, F,
                                         a.codes, e.kpad_f, e.kpad_f, a.ascale, st),
                "glu_rmsnorm_quant"));
  return wcheck(wfb_linear_i2s_residual(Ly.down, H, e.kpad_f, a.codes, m, e.kpad_f, a.ascale, Ly.scales + 6, 0.0f, a.x,
                                        g, H, a.x, g, H, st),
                "linear_residual (down)");
}

// Final RMSNorm + LM head on the pending hidden state dec.x[0]: first-max token into ctl[0] over the fp32
// logits (as the reference's std::max_element, bitnet_engine.cpp:774-779), logits stored (fp32) when `logits`.
int head(Engine& e, bool logits) {
  const Cfg& c = e.c;
  Acts& a = e.dec;
  const int g = e.gdt;
  if (e.head_q) {
    ECHECK(wcheck(wfb_rmsnorm_quant_i8(a.x, g, c.hidden, e.final_norm, g, c.rms_eps, 1, c.hidden, a.codes, e.kpad_h,
                                       e.kpad_h, a.ascale, e.s),
                  "rmsnorm_quant (head)"));
    return wcheck(wfb_linear_i2s_argmax(e.head_q, c.vocab, e.kpad_h, a.codes, 1, e.kpad_h, a.ascale, e.head_scale, 0.0f,
                                        logits ? e.logits : nullptr, WFB_F32, c.vocab, e.argmax_ws, e.ctl, e.s),
                  "LM head");
  }
  return wcheck(wfb_lm_head_argmax(a.x, g, c.hidden, e.final_norm, g, c.rms_eps, e.head_dense, g, c.hidden, 1, c.vocab,
                                   c.hidden, logits ? static_cast<float*>(e.logits) : nullptr, c.vocab, e.argmax_ws,
                                   e.ctl, e.s),
                "LM head");
}

// Embedding of the token ctl[0], every layer at position ctl[1], commit.
int body(Engine& e) {
  const Cfg& c = e.c;
  Acts& a = e.dec;
  HCHECK(wfb::launch_embed_rows(e.embed, c.vocab, (int)c.hidden, (int)e.es, e.ctl, 1, a.x, e.s), "embedding");
  for (const Layer& Ly : e.L) ECHECK(layer(e, Ly, a, 1, false));
  HCHECK(wfb::launch_commit(e.ctl, e.tokens, c.max_len, e.last_tok, a.x, e.ring, kRing, (int)c.hidden, (int)e.es, e.s),
         "commit");
  return 0;
}

int greedy_step(Engine& e) {
  ECHECK(head(e, false));
  return body(e);
}

template <typename Fn>
int capture(Engine& e, Fn fn, hipGraphExec_t* out) {
  HCHECK(hipStreamBeginCapture(e.s, hipStreamCaptureModeThreadLocal), "graph capture");
  const int st = fn(e);
  hipGraph_t g = nullptr;
  const hipError_t ce = hipStreamEndCapture(e.s, &g);
  if (st != 0) {
    if (ce == hipSuccess && g) (void)hipGraphDestroy(g);
    return st;
  }
  if (ce != hipSuccess) return hipfail(ce, "graph capture");
  const hipError_t ie = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (ie != hipSuccess) return hipfail(ie, "graph instantiate");
  return 0;
}

int sync(Engine& e, const char* what) {
  HCHECK(hipStreamSynchronize(e.s), what);
  return 0;
}

// ctl[i] = value (host -> device through the pinned mirror; the caller synchronises before reuse).
int set_ctl(Engine& e, int i, int64_t v) {
  e.ctl_h[i] = v;
  HCHECK(hipMemcpyAsync(e.ctl + i, e.ctl_h + i, sizeof(int64_t), hipMemcpyHostToDevice, e.s), "control upload");
  return 0;
}

int prefill(Engine& e, const int32_t* ids, int64_t n) {
  const Cfg& c = e.c;
  if (n < 1) return efail("num_tokens must be >= 1");
  if (!ids) return efail("input_ids is NULL");
  if (n > c.max_len) return efail("prompt of " + std::to_string(n) + " tokens exceeds max_seq_len " +
                                  std::to_string(c.max_len));
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= c.vocab) return efail("token id " + std::to_string(ids[i]) + " out of range");
  e.have_hidden = false;
  e.seq_len = 0;
  if (n > e.pre.cap) {
    // Grow the prompt buffers. The old set is released first (no peak of both); the new set and its pinned
    // id buffer are committed only when every allocation succeeded, so a failure leaves no buffers (cap 0,
    // ids_h NULL) and a later prompt of any length allocates again.
    ECHECK(sync(e, "prefill"));
    const int64_t cap = std::min<int64_t>(c.max_len, std::max<int64_t>(n, 2 * e.pre.cap));
    free_acts(e, e.pre);
    if (e.ids_h) (void)hipHostFree(e.ids_h);
    e.ids_h = nullptr;
    Acts grown;
    ECHECK(alloc_acts(e, grown, cap));
    int64_t* ids_h = nullptr;
    int st = alloc_gate("hipHostMalloc");
    if (st == 0) {
      const hipError_t he = hipHostMalloc((void**)&ids_h, cap * sizeof(int64_t), hipHostMallocDefault);
      if (he != hipSuccess) st = hipfail(he, "hipHostMalloc");
    }
    if (st != 0) {
      free_acts(e, grown);
      return st;
    }
    e.pre = grown;
    e.ids_h = ids_h;
  }
  Acts& a = e.pre;
  for (int64_t i = 0; i < n; ++i) e.ids_h[i] = ids[i];
  HCHECK(hipMemcpyAsync(a.ids, e.ids_h, n * sizeof(int64_t), hipMemcpyHostToDevice, e.s), "prompt upload");
  HCHECK(wfb::launch_embed_rows(e.embed, c.vocab, (int)c.hidden, (int)e.es, a.ids, n, a.x, e.s), "embedding");
  for (const Layer& Ly : e.L) ECHECK(layer(e, Ly, a, n, true));
  HCHECK(hipMemcpyAsync(e.dec.x, at(e, a.x, (n - 1) * c.hidden), c.hidden * e.es, hipMemcpyDeviceToDevice, e.s),
         "hidden copy");
  ECHECK(sync(e, "prefill"));
  e.seq_len = n;
  e.have_hidden = true;
  return 0;
}

// ---- top-p sampling (the reference's sample_top_p, bitnet_engine.cpp:208-253, 782-788) ----------

int32_t sample_top_p(const float* logits, int64_t n, float temperature, float top_p, std::mt19937& rng,
                     std::vector<float>& probs, std::vector<std::pair<float, int32_t>>& order) {
  probs.resize((size_t)n);
  for (int64_t v = 0; v < n; ++v) probs[v] = logits[v] / temperature;
  float mx = probs[0];
  for (int64_t v = 1; v < n; ++v) mx = std::max(mx, probs[v]);
  float sum = 0.0f;
  for (int64_t v = 0; v < n; ++v) {
    probs[v] = std::exp(probs[v] - mx);
    sum += probs[v];
  }
  for (int64_t v = 0; v < n; ++v) probs[v] /= sum;
  order.clear();
  order.reserve((size_t)n);
  for (int64_t v = 0; v < n; ++v) order.emplace_back(probs[v], (int32_t)v);
  std::sort(order.begin(), order.end(), [](const std::pair<float, int32_t>& x, const std::pair<float, int32_t>& y) {
    return x.first > y.first;
  });
  const float p = top_p > 0.0f ? top_p : 1.0f;
  float run = 0.0f;
  int64_t keep = 0;
  for (int64_t i = 0; i < n; ++i) {
    run += order[i].first;
    if (run >= p) {
      keep = i + 1;
      break;
    }
  }
  // float rounding can leave the whole sum below top_p: then the nucleus is every token (the reference
  // keeps only the first one there, turning top_p = 1 sampling into greedy picks)
  if (keep == 0) keep = n;
  std::uniform_real_distribution<float> u(0.0f, run);
  const float r = u(rng);
  float acc = 0.0f;
  for (int64_t i = 0; i < keep; ++i) {
    acc += order[i].first;
    if (r < acc) return order[i].second;
  }
  return order[0].second;
}

// Host float logits of the last head replay.
// Head with logits (fp32 for either head), host sample: the picked token (not yet run through the model).
int pick_sampled(Engine& e, float temperature, float top_p, int32_t* tok) {
  HCHECK(hipGraphLaunch(e.g_head, e.s), "graph launch");
  HCHECK(hipMemcpyAsync(e.logits_h, e.logits, (size_t)e.c.vocab * 4, hipMemcpyDeviceToHost, e.s), "logits download");
  ECHECK(sync(e, "head"));
  std::vector<float> probs;
  std::vector<std::pair<float, int32_t>> order;
  *tok = sample_top_p(static_cast<const float*>(e.logits_h), e.c.vocab, temperature, top_p, e.rng, probs, order);
  return 0;
}

// Run the host-chosen token at `pos` (embedding, layers, commit).
int run_token(Engine& e, int32_t tok, int64_t pos) {
  ECHECK(set_ctl(e, 0, tok));
  ECHECK(set_ctl(e, 1, pos));
  ECHECK(set_ctl(e, 2, 0));
  HCHECK(hipGraphLaunch(e.g_body, e.s), "graph launch");
  return sync(e, "decode step");
}

bool is_eos(const Engine& e, int64_t tok) {
  return std::find(e.c.eos.begin(), e.c.eos.end(), tok) != e.c.eos.end();
}

int create(Engine& e, const char* path, const BitNetConfig* user) {
  ModelFile f;
  ECHECK(open_model(path, f));
  Cfg& c = e.c;
  const std::string& js = f.json;
  double v = 0;
  // every size of the config is a positive integer well inside 32 bits (products of them stay in 64)
  auto in_range = [](double x) { return x >= 1.0 && x <= (double)(1 << 30); };
  auto req = [&](const char* key, int64_t& out) -> int {
    if (!json_num(js, key, v) || !in_range(v))
      return efail(std::string("Invalid config: ") + key + " missing, 0 or out of range");
    out = (int64_t)v;
    return 0;
  };
  if (!json_num(js, "vocab_size", v) || v <= 0 || !json_num(js, "hidden_size", v) || v <= 0)
    return efail("Invalid config: vocab_size or hidden_size is 0");
  ECHECK(req("vocab_size", c.vocab));
  ECHECK(req("hidden_size", c.hidden));
  ECHECK(req("intermediate_size", c.inter));
  ECHECK(req("num_hidden_layers", c.layers));
  ECHECK(req("num_attention_heads", c.heads));
  c.kv_heads = json_num(js, "num_key_value_heads", v) && in_range(v) ? (int64_t)v : c.heads;
  c.head_dim = json_num(js, "head_dim", v) && in_range(v) ? (int64_t)v : c.hidden / c.heads;
  if (json_num(js, "rope_theta", v) && v > 0 && std::isfinite(v)) c.theta = v;
  if (json_num(js, "rms_norm_eps", v) && v >= 0 && v < 1) c.rms_eps = (float)v;
  if (json_num(js, "subln_eps", v) && v >= 0 && v < 1) c.subln_eps = (float)v;
  c.max_len = json_num(js, "max_position_embeddings", v) && in_range(v) ? (int64_t)v : 4096;
  if (user && user->max_seq_len > 0) c.max_len = user->max_seq_len;
  if (c.vocab > (1 << 26) || c.layers > 4096) return efail("Invalid config: vocab_size or num_hidden_layers too large");
  const std::string act = json_raw(js, "hidden_act");
  if (act.empty() || act == "\"silu\"") {
    c.act = WFB_ACT_SILU;
  } else if (act == "\"relu2\"") {
    c.act = WFB_ACT_RELU2;
  } else {
    return efail("hidden_act " + act + " not supported (silu, relu2)");
  }
  const std::string eos = json_raw(js, "eos_token_id");
  for (size_t p = 0; p < eos.size();) {  // an id or a list of ids
    while (p < eos.size() && !(eos[p] == '-' || (eos[p] >= '0' && eos[p] <= '9'))) ++p;
    if (p >= eos.size()) break;
    char* end = nullptr;
    const long long id = std::strtoll(eos.c_str() + p, &end, 10);
    if (end == eos.c_str() + p) {  // a lone '-'
      ++p;
      continue;
    }
    c.eos.push_back(id);
    p = (size_t)(end - eos.c_str());
  }
  // what the kernels take
  if (c.head_dim != 64 && c.head_dim != 128) return efail("head_dim must be 64 or 128");
  if (c.heads % c.kv_heads != 0 || c.heads / c.kv_heads > 8)
    return efail("num_attention_heads must be 1..8 times num_key_value_heads");
  if (c.hidden % 8 != 0 || c.inter % 8 != 0 || c.hidden > WFB_NORM_MAX_H || c.inter > WFB_NORM_MAX_H ||
      c.qd() > WFB_NORM_MAX_H)
    return efail("hidden_size, intermediate_size and heads x head_dim must be multiples of 8 up to 16384");
  if (c.max_len < 1 || c.max_len > (1 << 20)) return efail("max_seq_len out of range (1 .. 1048576)");
  e.kpad_h = (c.hidden + WFB_QK_I2S - 1) / WFB_QK_I2S * WFB_QK_I2S;
  e.kpad_qd = (c.qd() + WFB_QK_I2S - 1) / WFB_QK_I2S * WFB_QK_I2S;
  e.kpad_f = (c.inter + WFB_QK_I2S - 1) / WFB_QK_I2S * WFB_QK_I2S;
  e.kmax = std::max(e.kpad_h, std::max(e.kpad_qd, e.kpad_f));
  e.seg_qkv[0] = c.qd();
  e.seg_qkv[1] = e.seg_qkv[2] = c.kvd();
  ECHECK(check_tensors(f, c));  // the whole file, before anything touches the GPU
  {
    const std::string td = json_raw(js, "torch_dtype");
    const TensorRec* emb = f.find("model.embed_tokens.weight");
    const bool fp32 = td.empty() ? emb->dtype == 1 : td == "\"float32\"";
    e.gdt = fp32 ? WFB_F32 : WFB_BF16;
    e.es = fp32 ? 4 : 2;
  }

  HCHECK(hipGetDevice(&e.device), "hipGetDevice");
  HCHECK(hipStreamCreateWithFlags(&e.s, hipStreamNonBlocking), "hipStreamCreate");
  Uploader up(e);
  const size_t scratch_bytes = 32u << 20;
  void* scratch = nullptr;
  ECHECK(dalloc_bytes(e, scratch, scratch_bytes));

  const int64_t H = c.hidden, F = c.inter, qd = c.qd(), kvd = c.kvd(), V = c.vocab;
  ECHECK(galloc(e, e.embed, V * H));
  ECHECK(load_floats(e, up, f, "model.embed_tokens.weight", V * H, e.embed, false, scratch, scratch_bytes));
  e.L.resize((size_t)c.layers);
  for (int64_t i = 0; i < c.layers; ++i) {
    Layer& Ly = e.L[(size_t)i];
    const std::string pre = "model.layers." + std::to_string(i) + ".";
    std::vector<float> sc(7, 1.0f);
    ECHECK(dalloc(e, Ly.qkv, c.nqkv() * e.kpad_h / 4));
    ECHECK(dalloc(e, Ly.o, H * e.kpad_qd / 4));
    ECHECK(dalloc(e, Ly.gu, 2 * F * e.kpad_h / 4));
    ECHECK(dalloc(e, Ly.down, H * e.kpad_f / 4));
    ECHECK(dalloc(e, Ly.scales, 8));
    ECHECK(load_packed(up, f, pre + "self_attn.q_proj.weight", qd, H, Ly.qkv, sc, 0));
    ECHECK(load_packed(up, f, pre + "self_attn.k_proj.weight", kvd, H, Ly.qkv + qd * e.kpad_h / 4, sc, 1));
    ECHECK(load_packed(up, f, pre + "self_attn.v_proj.weight", kvd, H, Ly.qkv + (qd + kvd) * e.kpad_h / 4,
                       sc, 2));
    ECHECK(load_packed(up, f, pre + "self_attn.o_proj.weight", H, qd, Ly.o, sc, 3));
    ECHECK(load_packed(up, f, pre + "mlp.gate_proj.weight", F, H, Ly.gu, sc, 4));
    ECHECK(load_packed(up, f, pre + "mlp.up_proj.weight", F, H, Ly.gu + F * e.kpad_h / 4, sc, 5));
    ECHECK(load_packed(up, f, pre + "mlp.down_proj.weight", H, F, Ly.down, sc, 6));
    ECHECK(up.put(Ly.scales, reinterpret_cast<const uint8_t*>(sc.data()), 7 * sizeof(float)));
    ECHECK(galloc(e, Ly.in_norm, H));
    ECHECK(galloc(e, Ly.post_norm, H));
    ECHECK(galloc(e, Ly.attn_sub, qd));
    ECHECK(galloc(e, Ly.ffn_sub, F));
    ECHECK(load_floats(e, up, f, pre + "input_layernorm.weight", H, Ly.in_norm, false, scratch, scratch_bytes));
    ECHECK(load_floats(e, up, f, pre + "post_attention_layernorm.weight", H, Ly.post_norm, false, scratch,
                       scratch_bytes));
    ECHECK(load_floats(e, up, f, pre + "self_attn.attn_sub_norm.weight", qd, Ly.attn_sub, true, scratch, scratch_bytes));
    ECHECK(load_floats(e, up, f, pre + "mlp.ffn_sub_norm.weight", F, Ly.ffn_sub, true, scratch, scratch_bytes));
    const int64_t cache = c.kv_heads * c.max_len * c.head_dim;
    ECHECK(galloc(e, Ly.kc, cache));
    ECHECK(galloc(e, Ly.vc, cache));
    HCHECK(hipMemsetAsync(Ly.kc, 0, cache * e.es, e.s), "cache clear");
    HCHECK(hipMemsetAsync(Ly.vc, 0, cache * e.es, e.s), "cache clear");
  }
  ECHECK(galloc(e, e.final_norm, H));
  ECHECK(load_floats(e, up, f, "model.norm.weight", H, e.final_norm, false, scratch, scratch_bytes));
  if (const TensorRec* t = f.find("lm_head.weight")) {
    if (t->dtype == 0) {
      std::vector<float> sc(1, 1.0f);
      ECHECK(dalloc(e, e.head_q, V * e.kpad_h / 4));
      ECHECK(dalloc(e, e.head_scale, 1));
      ECHECK(load_packed(up, f, "lm_head.weight", V, H, e.head_q, sc, 0));
      ECHECK(up.put(e.head_scale, reinterpret_cast<const uint8_t*>(sc.data()), sizeof(float)));
    } else {
      ECHECK(galloc(e, e.head_dense, V * H));
      ECHECK(load_floats(e, up, f, "lm_head.weight", V * H, e.head_dense, false, scratch, scratch_bytes));
    }
  } else {
    e.head_dense = e.embed;  // tied
  }
  // rotary tables, decode buffers, graph state
  {
    std::vector<float> cs((size_t)(c.max_len * c.head_dim / 2)), sn(cs.size());
    ECHECK(wcheck(wfb_rope_tables(c.theta, c.head_dim, c.max_len, cs.data(), sn.data()), "rope tables"));
    ECHECK(dalloc(e, e.rope_cos, cs.size()));
    ECHECK(dalloc(e, e.rope_sin, sn.size()));
    ECHECK(up.put(e.rope_cos, reinterpret_cast<const uint8_t*>(cs.data()), cs.size() * 4));
    ECHECK(up.put(e.rope_sin, reinterpret_cast<const uint8_t*>(sn.data()), sn.size() * 4));
    ECHECK(sync(e, "upload"));
  }
  dfree(e, scratch);
  ECHECK(alloc_acts(e, e.dec, 1));
  ECHECK(dalloc(e, e.attn_ws, (size_t)WFB_ATTN_WS(1, c.heads, c.head_dim, c.max_len)));
  ECHECK(dalloc(e, e.argmax_ws, (size_t)WFB_ARGMAX_WS(1, V)));
  ECHECK(dalloc(e, e.ctl, 4));
  ECHECK(dalloc(e, e.tokens, c.max_len));
  ECHECK(dalloc(e, e.last_tok, 1));
  ECHECK(galloc(e, e.ring, kRing * H));
  ECHECK(galloc(e, e.x_start, H));
  if (e.gdt == WFB_F32) {
    std::vector<int64_t> iota((size_t)c.max_len);
    for (int64_t i = 0; i < c.max_len; ++i) iota[(size_t)i] = i;
    ECHECK(dalloc(e, e.iota, c.max_len));
    HCHECK(hipMemcpy(e.iota, iota.data(), iota.size() * sizeof(int64_t), hipMemcpyHostToDevice), "positions upload");
  }
  ECHECK(dalloc_bytes(e, e.logits, V * 4));
  HCHECK(hipHostMalloc((void**)&e.ctl_h, 4 * sizeof(int64_t), hipHostMallocDefault), "hipHostMalloc");
  HCHECK(hipHostMalloc(&e.logits_h, V * 4, hipHostMallocDefault), "hipHostMalloc");
  HCHECK(hipHostMalloc((void**)&e.tokens_h, kChunk * sizeof(int32_t), hipHostMallocDefault), "hipHostMalloc");
  HCHECK(hipMemsetAsync(e.dec.x, 0, H * e.es, e.s), "clear");
  for (int i = 0; i < 3; ++i) ECHECK(set_ctl(e, i, 0));
  // one eager step (position 0 of every cache, rewritten by the first prompt) before the captures
  ECHECK(head(e, true));
  ECHECK(body(e));
  ECHECK(sync(e, "warm-up"));
  ECHECK(capture(e, greedy_step, &e.g_greedy));
  ECHECK(capture(e, [](Engine& en) { return head(en, true); }, &e.g_head));
  ECHECK(capture(e, body, &e.g_body));
  e.seq_len = 0;
  e.have_hidden = false;
  return 0;
}

int generate(Engine& e, const int32_t* ids, int32_t n, const SamplingParams* p, GenerationResult* res) {
  if (!p) return efail("params is NULL");
  if (!res) return efail("result is NULL");
  res->output_ids = nullptr;
  res->num_tokens = 0;
  res->logits = nullptr;
  res->logits_size = 0;
  const int64_t max_new = std::max<int32_t>(p->max_tokens, 0);
  if (n < 1) return efail("num_input_tokens must be >= 1");
  if ((int64_t)n + max_new > e.c.max_len)
    return efail("num_input_tokens + max_tokens (" + std::to_string((int64_t)n + max_new) + ") exceeds max_seq_len " +
                 std::to_string(e.c.max_len));
  ECHECK(prefill(e, ids, n));
  e.have_hidden = false;  // until the steps below complete: a failure leaves no pending state
  std::vector<int32_t> out;
  out.reserve((size_t)max_new);
  if (p->temperature <= 0.0f) {
    ECHECK(set_ctl(e, 1, n));
    ECHECK(set_ctl(e, 2, 0));
    HCHECK(hipMemcpyAsync(e.x_start, e.dec.x, e.c.hidden * e.es, hipMemcpyDeviceToDevice, e.s), "hidden copy");
    int64_t eos_at = -1;
    while ((int64_t)out.size() < max_new && eos_at < 0) {
      const int64_t c0 = (int64_t)out.size();
      const int64_t len = std::min<int64_t>(kChunk, max_new - c0);
      for (int64_t r = 0; r < len; ++r) HCHECK(hipGraphLaunch(e.g_greedy, e.s), "graph launch");
      HCHECK(hipMemcpyAsync(e.tokens_h, e.tokens + c0, len * sizeof(int32_t), hipMemcpyDeviceToHost, e.s),
             "token download");
      ECHECK(sync(e, "decode"));
      for (int64_t r = 0; r < len; ++r) {
        out.push_back(e.tokens_h[r]);
        if (is_eos(e, e.tokens_h[r])) {
          eos_at = c0 + r;
          break;
        }
      }
    }
    if (eos_at >= 0) {
      // the reference stops before running the EOS token: state after token eos_at - 1
      const void* src = eos_at == 0 ? e.x_start : at(e, e.ring, ((eos_at - 1) % kRing) * e.c.hidden);
      HCHECK(wfb::launch_copy_row(src, e.dec.x, (int)e.c.hidden, (int)e.es, e.s), "hidden restore");
      ECHECK(sync(e, "decode"));
      e.seq_len = n + eos_at;
    } else {
      e.seq_len = n + (int64_t)out.size();
    }
  } else {
    for (int64_t i = 0; i < max_new; ++i) {
      int32_t tok = 0;
      ECHECK(pick_sampled(e, p->temperature, p->top_p, &tok));
      out.push_back(tok);
      if (is_eos(e, tok)) break;
      ECHECK(run_token(e, tok, e.seq_len));
      e.seq_len += 1;
    }
  }
  e.have_hidden = true;
  res->num_tokens = (int32_t)out.size();
  res->output_ids = static_cast<int32_t*>(std::malloc(std::max<size_t>(out.size(), 1) * sizeof(int32_t)));
  if (!res->output_ids) return efail("out of host memory");
  if (!out.empty()) std::memcpy(res->output_ids, out.data(), out.size() * sizeof(int32_t));
  return 0;
}

int decode_step(Engine& e, int32_t position, const SamplingParams* p, int32_t* output_id) {
  if (!p) return efail("params is NULL");
  if (!output_id) return efail("output_id is NULL");
  if (!e.have_hidden) return efail("no prompt has been run (call bitnet_prefill first)");
  if (position < 0 || position >= e.c.max_len)
    return efail("position " + std::to_string(position) + " outside [0, max_seq_len " + std::to_string(e.c.max_len) +
                 ")");
  e.have_hidden = false;  // until the step completes: a failure leaves no pending state
  if (p->temperature <= 0.0f) {
    ECHECK(set_ctl(e, 1, position));
    ECHECK(set_ctl(e, 2, 0));
    HCHECK(hipGraphLaunch(e.g_greedy, e.s), "graph launch");
    HCHECK(hipMemcpyAsync(e.tokens_h, e.last_tok, sizeof(int32_t), hipMemcpyDeviceToHost, e.s), "token download");
    ECHECK(sync(e, "decode step"));
    *output_id = e.tokens_h[0];
  } else {
    int32_t tok = 0;
    ECHECK(pick_sampled(e, p->temperature, p->top_p, &tok));
    ECHECK(run_token(e, tok, position));
    *output_id = tok;
  }
  e.seq_len = (int64_t)position + 1;
  e.have_hidden = true;
  return 0;
}

// Every entry point runs on the engine's device and gives the calling thread its own current device back.
class DeviceScope {
 public:
  int enter(const Engine* e) {
    if (!e) return efail("Engine not initialized");
    HCHECK(hipGetDevice(&prev_), "hipGetDevice");
    if (prev_ != e->device) {
      HCHECK(hipSetDevice(e->device), "hipSetDevice");
      restore_ = true;
    }
    return 0;
  }
  ~DeviceScope() {
    if (restore_) (void)hipSetDevice(prev_);
  }

 private:
  int prev_ = 0;
  bool restore_ = false;
};

}  // namespace

extern "C" {

BitNetEngine* bitnet_engine_create(const char* model_path, const BitNetConfig* config) {
  Engine* e = new (std::nothrow) Engine();
  if (!e) {
    efail("out of host memory");
    return nullptr;
  }
  if (create(*e, model_path, config) != 0) {
    delete e;
    return nullptr;
  }
  return e;
}

void bitnet_engine_destroy(BitNetEngine* engine) {
  if (!engine) return;
  DeviceScope dev;
  (void)dev.enter(engine);
  delete engine;
}

const char* bitnet_get_error(void) { return g_eng_err.c_str(); }

int bitnet_generate(BitNetEngine* engine, const int32_t* input_ids, int32_t num_input_tokens,
                    const SamplingParams* params, GenerationResult* result) {
  DeviceScope dev;
  if (dev.enter(engine) != 0) return -1;
  return generate(*engine, input_ids, num_input_tokens, params, result) == 0 ? 0 : -1;
}

int bitnet_prefill(BitNetEngine* engine, const int32_t* input_ids, int32_t num_tokens) {
  DeviceScope dev;
  if (dev.enter(engine) != 0) return -1;
  return prefill(*engine, input_ids, num_tokens) == 0 ? 0 : -1;
}

int bitnet_decode_step(BitNetEngine* engine, int32_t position, const SamplingParams* params, int32_t* output_id) {
  DeviceScope dev;
  if (dev.enter(engine) != 0) return -1;
  return decode_step(*engine, position, params, output_id) == 0 ? 0 : -1;
}

void bitnet_reset_cache(BitNetEngine* engine) {
  if (!engine) return;
  engine->seq_len = 0;
  engine->have_hidden = false;
}

int32_t bitnet_vocab_size(BitNetEngine* engine) { return engine ? (int32_t)engine->c.vocab : 0; }
int32_t bitnet_hidden_size(BitNetEngine* engine) { return engine ? (int32_t)engine->c.hidden : 0; }
int32_t bitnet_num_layers(BitNetEngine* engine) { return engine ? (int32_t)engine->c.layers : 0; }
int32_t bitnet_max_seq_len(BitNetEngine* engine) { return engine ? (int32_t)engine->c.max_len : 0; }
int bitnet_get_num_kv_heads(BitNetEngine* engine) { return engine ? (int)engine->c.kv_heads : 0; }

void bitnet_free_result(GenerationResult* result) {
  if (!result) return;
  std::free(result->output_ids);
  std::free(result->logits);
  result->output_ids = nullptr;
  result->logits = nullptr;
}

int wfb_engine_fail_alloc_after(int64_t n) {
  g_fail_alloc_after.store(n < 0 ? -1 : n);
  return 0;
}

int wfb_engine_sample_top_p(const float* logits, int64_t n, float temperature, float top_p, uint32_t seed,
                            int32_t draws, int32_t* out) {
  if (!logits || (draws > 0 && !out) || n < 1 || !(temperature > 0.0f) || draws < 0)
    return efail("wfb_engine_sample_top_p: bad arguments");
  std::mt19937 rng(seed);
  std::vector<float> probs;
  std::vector<std::pair<float, int32_t>> order;
  for (int32_t i = 0; i < draws; ++i) out[i] = sample_top_p(logits, n, temperature, top_p, rng, probs, order);
  return 0;
}

}  // extern "C"
