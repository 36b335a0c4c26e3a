// Host-side AddressSanitizer driver for the C ABI of libwfbitnet (built with the host-only ASan library by
// wrinklefree-monorepo_amd/_build.py build_asan; run by tests/test_asan_host.py, no GPU needed).
//
// Exercises every path that runs on the host before any GPU work:
//  * argument validation of the op entry points (each call below must be refused with WFB_EINVAL and a
//    message, without touching the fake device pointers it is given);
//  * wfb_rope_tables on host buffers;
//  * the native engine's model loader on the SGLBITNT files named on the command line: the file itself,
//    every truncation inside its headers and a sample inside its data, and corrupted header fields and
//    config texts -- each create must return NULL with a message (without a GPU a well-formed file fails
//    at the first HIP call) and ASan must see no bad access;
//  * the NULL-engine contract and the top-p sampler.
// Exit status 0 when every expectation held; ASan aborts the process on a memory error.
#include <fcntl.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "wfbitnet.h"
#include "wfbitnet_engine.h"

static int g_fail = 0;
static void expect(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s\n", what);
    ++g_fail;
  }
}

static void* fake(uintptr_t a) { return reinterpret_cast<void*>(a); }  // never dereferenced on the host

static void refused(int st, const char* what) {
  expect(st == WFB_EINVAL && std::strlen(wfb_last_error()) > 0, what);
}

static void op_validation() {
  const uint8_t* W = static_cast<const uint8_t*>(fake(0x1000));
  const int8_t* A = static_cast<const int8_t*>(fake(0x2000));
  void* O = fake(0x3000);
  refused(wfb_linear_i2s(W, 256, 200, A, 1, 200, nullptr, nullptr, 1.0f, nullptr, 0, O, WFB_BF16, 256, nullptr, nullptr),
          "K % 128");
  refused(wfb_linear_i2s(nullptr, 256, 256, A, 1, 256, nullptr, nullptr, 1.0f, nullptr, 0, O, WFB_BF16, 256, nullptr,
                         nullptr),
          "null weights");
  refused(wfb_linear_i2s(static_cast<const uint8_t*>(fake(0x1008)), 256, 256, A, 1, 256, nullptr, nullptr, 1.0f,
                         nullptr, 0, O, WFB_BF16, 256, nullptr, nullptr),
          "misaligned weights");
  refused(wfb_linear_i2s(W, 256, 256, A, 2, 100, nullptr, nullptr, 1.0f, nullptr, 0, O, WFB_BF16, 256, nullptr, nullptr),
          "activation stride");
  refused(wfb_linear_i2s(W, 256, 256, A, 1, 256, nullptr, nullptr, 1.0f, nullptr, 0, O, WFB_F16, 256, nullptr, nullptr),
          "output dtype");
  refused(wfb_linear_i2s(W, 256, 256, A, 1, 256, nullptr, nullptr, 1.0f, nullptr, 0, O, WFB_BF16, 10, nullptr, nullptr),
          "output stride");
  refused(wfb_linear_i2s(W, 256, 256, A, 1, 256, nullptr, nullptr, 1.0f, nullptr, 0, nullptr, WFB_BF16, 256, nullptr,
                         nullptr),
          "no output");
  refused(wfb_gemv_i2s(W, 256, 256, A, 4, 256, nullptr, nullptr, 1.0f, nullptr, 0, O, WFB_BF16, 256, nullptr, nullptr),
          "GEMV rows");
  refused(wfb_linear_i2s(W, (int64_t)1 << 40, 256, A, 1, 256, nullptr, nullptr, 1.0f, nullptr, 0, O, WFB_BF16,
                         (int64_t)1 << 40, nullptr, nullptr),
          "huge N");
  const int64_t bad_rows[3] = {100, 100, 57};
  refused(wfb_linear_i2s_segmented(W, 257, 256, 3, bad_rows, static_cast<const float*>(fake(0x4000)), A, 1, 256,
                                   nullptr, nullptr, 0, O, WFB_BF16, 257, nullptr, nullptr),
          "segment rows");
  refused(wfb_linear_i2s_segmented(W, 256, 256, 9, bad_rows, static_cast<const float*>(fake(0x4000)), A, 1, 256,
                                   nullptr, nullptr, 0, O, WFB_BF16, 256, nullptr, nullptr),
          "segment count");
  refused(wfb_rmsnorm_quant_i8(fake(0x5000), WFB_BF16, 100, nullptr, WFB_F32, 1e-6f, 1, 100, static_cast<int8_t*>(fake(0x7000)), 128, 128,
                               static_cast<float*>(fake(0x6000)), nullptr),
          "norm row length % 8");
  refused(wfb_rmsnorm_quant_i8(fake(0x5000), WFB_BF16, 20000, nullptr, WFB_F32, 1e-6f, 1, 20000,
                               static_cast<int8_t*>(fake(0x7000)), 20096, 20096, static_cast<float*>(fake(0x6000)), nullptr),
          "norm row too long");
  refused(wfb_glu_rmsnorm_quant_i8(fake(0x5000), fake(0x5100), WFB_BF16, 256, 7, nullptr, WFB_F32, 1e-6f, 1, 256,
                                   static_cast<int8_t*>(fake(0x7000)), 256, 256, static_cast<float*>(fake(0x6000)), nullptr),
          "gated activation kind");
  const int64_t rows1[1] = {256};
  refused(wfb_rmsnorm_linear_i2s(fake(0x5000), WFB_BF16, 256, nullptr, WFB_F32, 1e-6f, 17, 256, W, 256, 256, 1, rows1,
                                 static_cast<const float*>(fake(0x4000)), nullptr, WFB_F32, 256, O, WFB_BF16, 256, nullptr),
          "fused norm rows");
  refused(wfb_rmsnorm_linear_i2s(fake(0x5000), WFB_BF16, 8192, nullptr, WFB_F32, 1e-6f, 2, 8192, W, 256, 8192, 1, rows1,
                                 static_cast<const float*>(fake(0x4000)), nullptr, WFB_F32, 256, O, WFB_BF16, 256, nullptr),
          "fused norm length at M 2");
  refused(wfb_rmsnorm_linear_i2s(fake(0x5000), WFB_BF16, 16392, nullptr, WFB_F32, 1e-6f, 1, 16392, W, 256, 16512, 1,
                                 rows1, static_cast<const float*>(fake(0x4000)), nullptr, WFB_F32, 256, O, WFB_BF16, 256,
                                 nullptr),
          "fused norm length past 16384");
  refused(wfb_linear_i2s_glu(W, 96, 256, A, 1, 256, nullptr, static_cast<const float*>(fake(0x4000)), WFB_ACT_SILU,
                             WFB_BF16, static_cast<float*>(fake(0x8000)), 48, nullptr),
          "gated half % 32");
  refused(wfb_gqa_decode_attention(fake(0x9000), 768, fake(0x9100), 256, fake(0x9200), 256, WFB_BF16, nullptr, nullptr,
                                   fake(0xa000), fake(0xb000), 64, static_cast<const int64_t*>(fake(0xc000)), 1, 8, 1,
                                   96, 0.1f, fake(0xd000), 768, nullptr, nullptr),
          "attention head_dim");
  refused(wfb_gqa_decode_attention(fake(0x9000), 1152, fake(0x9100), 64, fake(0x9200), 64, WFB_BF16, nullptr, nullptr,
                                   fake(0xa000), fake(0xb000), 64, static_cast<const int64_t*>(fake(0xc000)), 1, 18, 1,
                                   64, 0.1f, fake(0xd000), 1152, nullptr, nullptr),
          "attention group size");
  refused(wfb_gqa_prefill_attention(fake(0x9000), 512, fake(0x9100), 128, fake(0x9200), 128, WFB_F32, nullptr, nullptr,
                                    fake(0xa000), fake(0xb000), 64, 0, 1, 4, 4, 2, 64, 0.1f, fake(0xd000), 256, nullptr),
          "prefill attention dtype");
  refused(wfb_lm_head_argmax(fake(0x9000), WFB_BF16, 4096, nullptr, WFB_F32, 1e-5f, fake(0xa000), WFB_BF16, 4096, 16,
                             1000, 4096, nullptr, 1000, static_cast<uint64_t*>(fake(0xb000)),
                             static_cast<int64_t*>(fake(0xc000)), nullptr),
          "dense head size");
  // host-only entry point: the tables themselves
  std::vector<float> c(16 * 32), s(16 * 32);
  expect(wfb_rope_tables(10000.0, 64, 16, c.data(), s.data()) == WFB_OK && c[0] == 1.0f && s[0] == 0.0f,
         "rope tables");
  refused(wfb_rope_tables(10000.0, 63, 16, c.data(), s.data()), "rope head_dim");
  refused(wfb_rope_tables(0.0, 64, 16, c.data(), s.data()), "rope theta");
  refused(wfb_rope_tables(10000.0, 64, 16, nullptr, s.data()), "rope null");
}

// ---- engine loader --------------------------------------------------------------------------------

static std::vector<uint8_t> read_file(const char* path) {
  std::vector<uint8_t> d;
  FILE* f = std::fopen(path, "rb");
  if (!f) return d;
  std::fseek(f, 0, SEEK_END);
  d.resize((size_t)std::ftell(f));
  std::fseek(f, 0, SEEK_SET);
  if (std::fread(d.data(), 1, d.size(), f) != d.size()) d.clear();
  std::fclose(f);
  return d;
}

static std::string g_tmp;
static void write_tmp(const uint8_t* p, size_t n) {
  FILE* f = std::fopen(g_tmp.c_str(), "wb");
  if (n) std::fwrite(p, 1, n, f);
  std::fclose(f);
}

static int g_creates = 0;
// create on the bytes: NULL with a message expected (no GPU here); an engine is destroyed at once
static void try_create(const std::vector<uint8_t>& bytes, size_t n, const char* what) {
  write_tmp(bytes.data(), n);
  BitNetConfig cfg = {64, 0, 0};
  BitNetEngine* e = bitnet_engine_create(g_tmp.c_str(), &cfg);
  ++g_creates;
  if (e) {
    bitnet_engine_destroy(e);
  } else {
    expect(std::strlen(bitnet_get_error()) > 0, what);
  }
}

struct Field {
  size_t off, len;
};

// Header fields of an SGLBITNT file (magic, version, config length, count; per tensor name length, dtype,
// ndims, dims, scale flag, scale, byte count) and the tensor data ranges.
static bool layout(const std::vector<uint8_t>& b, std::vector<Field>& hdr, std::vector<Field>& data, size_t& cfg_off,
                   size_t& cfg_len) {
  size_t at = 0;
  auto u32 = [&](uint32_t& v) {
    if (at + 4 > b.size()) return false;
    std::memcpy(&v, b.data() + at, 4);
    hdr.push_back({at, 4});
    at += 4;
    return true;
  };
  hdr.push_back({0, 8});
  at = 8;
  uint32_t ver, clen, count;
  if (!u32(ver) || !u32(clen)) return false;
  cfg_off = at;
  cfg_len = clen;
  at += clen;
  if (!u32(count)) return false;
  for (uint32_t i = 0; i < count; ++i) {
    uint32_t nlen, dt, nd, hs;
    if (!u32(nlen)) return false;
    at += nlen;
    if (!u32(dt) || !u32(nd)) return false;
    for (uint32_t d = 0; d < nd; ++d) {
      uint32_t x;
      if (!u32(x)) return false;
    }
    if (!u32(hs)) return false;
    if (hs == 1) {
      uint32_t sc;
      if (!u32(sc)) return false;
    }
    uint64_t nb;
    if (at + 8 > b.size()) return false;
    std::memcpy(&nb, b.data() + at, 8);
    hdr.push_back({at, 8});
    at += 8;
    data.push_back({at, (size_t)nb});
    at += nb;
  }
  return at == b.size();
}

static void engine_loader(const char* path) {
  const std::vector<uint8_t> full = read_file(path);
  expect(!full.empty(), "model file readable");
  if (full.empty()) return;
  std::vector<Field> hdr, data;
  size_t cfg_off = 0, cfg_len = 0;
  expect(layout(full, hdr, data, cfg_off, cfg_len), "model file layout");
  try_create(full, full.size(), "whole file");
  // truncations: every cut inside a header field (and just after it), 8 inside each data range, inside the config
  std::vector<size_t> cuts;
  for (const Field& f : hdr)
    for (size_t k = 0; k <= f.len; ++k) cuts.push_back(f.off + k);
  for (const Field& f : data)
    for (size_t k = 1; k <= 8; ++k) cuts.push_back(f.off + f.len * k / 9);
  for (size_t k = 0; k < cfg_len; k += 7) cuts.push_back(cfg_off + k);
  for (size_t n : cuts)
    if (n < full.size()) try_create(full, n, "truncated file");
  // corrupt header fields: extreme values in every 4-byte field, each alone
  const uint32_t vals[] = {0u, 1u, 3u, 9u, 0x7fffffffu, 0xffffffffu, 0x80000000u};
  for (const Field& f : hdr) {
    if (f.len != 4) continue;
    for (uint32_t v : vals) {
      std::vector<uint8_t> b = full;
      std::memcpy(b.data() + f.off, &v, 4);
      try_create(b, b.size(), "corrupt field");
    }
  }
  for (const Field& f : hdr) {  // the 8-byte data sizes
    if (f.len != 8) continue;
    for (uint64_t v : {(uint64_t)0, (uint64_t)1 << 62, ~(uint64_t)0}) {
      std::vector<uint8_t> b = full;
      std::memcpy(b.data() + f.off, &v, 8);
      try_create(b, b.size(), "corrupt size");
    }
  }
  // random byte flips in the header region (seeded)
  std::mt19937 rng(1234);
  for (int i = 0; i < 400; ++i) {
    std::vector<uint8_t> b = full;
    const Field& f = hdr[rng() % hdr.size()];
    b[f.off + rng() % f.len] ^= (uint8_t)(1u << (rng() % 8));
    try_create(b, b.size(), "flipped header bit");
  }
  // config texts the parser must survive (the file is rebuilt around each)
  const char* cfgs[] = {
      "", "{", "}", "\"vocab_size\"", "{\"vocab_size\": }", "{\"vocab_size\": 1e400, \"hidden_size\": 64}",
      "{\"vocab_size\": -5, \"hidden_size\": 64}", "{\"vocab_size\": nan, \"hidden_size\": nan}",
      "{\"vocab_size\": 64, \"hidden_size\": 128, \"hidden_act\": \"", "{\"eos_token_id\": [1, -, 2,",
      "{\"vocab_size\": 64, \"hidden_size\": 128, \"intermediate_size\": 256, \"num_hidden_layers\": 1, "
      "\"num_attention_heads\": 2, \"head_dim\": 64, \"eos_token_id\": [-, 3], \"max_position_embeddings\": 9e18}",
      "{\"vocab_size\": 64, \"hidden_size\": 128, \"intermediate_size\": 256, \"num_hidden_layers\": 100000, "
      "\"num_attention_heads\": 2}",
  };
  for (const char* cj : cfgs) {
    const uint32_t len = (uint32_t)std::strlen(cj);
    std::vector<uint8_t> b(full.begin(), full.begin() + 12);  // magic and version
    b.insert(b.end(), reinterpret_cast<const uint8_t*>(&len), reinterpret_cast<const uint8_t*>(&len) + 4);
    b.insert(b.end(), cj, cj + len);
    b.insert(b.end(), full.begin() + cfg_off + cfg_len, full.end());
    try_create(b, b.size(), "config text");
  }
}

static void engine_contract() {
  SamplingParams p = {0.0f, 1.0f, 0, 1.0f, 4};
  GenerationResult r = {nullptr, 0, nullptr, 0};
  const int32_t ids[2] = {1, 2};
  int32_t out = 0;
  expect(bitnet_generate(nullptr, ids, 2, &p, &r) == -1, "generate NULL");
  expect(std::strcmp(bitnet_get_error(), "Engine not initialized") == 0, "NULL message");
  expect(bitnet_prefill(nullptr, ids, 2) == -1, "prefill NULL");
  expect(bitnet_decode_step(nullptr, 0, &p, &out) == -1, "decode NULL");
  expect(bitnet_vocab_size(nullptr) == 0 && bitnet_hidden_size(nullptr) == 0 && bitnet_num_layers(nullptr) == 0 &&
             bitnet_max_seq_len(nullptr) == 0 && bitnet_get_num_kv_heads(nullptr) == 0,
         "sizes of NULL");
  bitnet_reset_cache(nullptr);
  bitnet_engine_destroy(nullptr);
  bitnet_free_result(nullptr);
  r.output_ids = static_cast<int32_t*>(std::malloc(16));
  bitnet_free_result(&r);
  expect(r.output_ids == nullptr && r.logits == nullptr, "free_result clears");
  expect(bitnet_engine_create(nullptr, nullptr) == nullptr, "create NULL path");
}

static void sampler() {
  std::mt19937 rng(5);
  std::normal_distribution<float> nd(0.0f, 3.0f);
  for (int n : {1, 2, 17, 1000, 50000}) {
    std::vector<float> logits((size_t)n);
    for (float& x : logits) x = nd(rng);
    std::vector<int32_t> out(64, -1);
    for (float t : {0.3f, 1.0f, 4.0f})
      for (float tp : {0.0f, 0.5f, 0.95f, 1.0f}) {
        expect(wfb_engine_sample_top_p(logits.data(), n, t, tp, 42, 64, out.data()) == 0, "sampler status");
        for (int32_t v : out) expect(v >= 0 && v < n, "sampled id in range");
      }
  }
  float one = 1.0f;
  int32_t o = 0;
  expect(wfb_engine_sample_top_p(&one, 0, 1.0f, 1.0f, 1, 1, &o) == -1, "sampler n 0");
  expect(wfb_engine_sample_top_p(&one, 1, 0.0f, 1.0f, 1, 1, &o) == -1, "sampler temperature 0");
  expect(wfb_engine_sample_top_p(nullptr, 1, 1.0f, 1.0f, 1, 1, &o) == -1, "sampler NULL");
}

int main(int argc, char** argv) {
  char tmpl[] = "/tmp/wfb_asan_XXXXXX";
  const int fd = mkstemp(tmpl);
  if (fd < 0) return 2;
  close(fd);
  g_tmp = tmpl;
  op_validation();
  engine_contract();
  sampler();
  for (int i = 1; i < argc; ++i) engine_loader(argv[i]);
  unlink(g_tmp.c_str());
  std::printf("abi_driver: %d engine creates, %d failures\n", g_creates, g_fail);
  return g_fail == 0 ? 0 : 1;
}
