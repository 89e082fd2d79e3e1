// C ABI of the MI355X ProteinMPNN v_48_020 design path (include/hkbs_pmpnn.h).
//
// Host responsibilities: parse the safetensors weight package, pack the
// weights into the device layouts the kernels read (one upload per context),
// validate requests with the reference's rules, compute decoding orders on
// the host (bit-exact with the reference's libm-based routine), manage a
// grow-only device workspace and enqueue the kernels on the context stream.
#include "../../include/hkbs_pmpnn.h"
#include "host_status.hpp"
#include "pmpnn_internal.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <type_traits>
#include <numeric>
#include <string>
#include <vector>

namespace {

using namespace hkbs;

thread_local const char* g_last_error = "";

hkbs_status fail(hkbs_status code, const char* detail) {
  g_last_error = detail;
  return code;
}

// ---------------------------------------------------------------- JSON ----
// Minimal JSON reader for the safetensors header.
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::map<std::string, Json> obj;
};

struct JsonParser {
  const char* p;
  const char* end;
  bool ok = true;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end - p) < n || std::strncmp(p, s, n) != 0) return false;
    p += n;
    return true;
  }
  std::string string() {
    std::string out;
    if (p >= end || *p != '"') {
      ok = false;
      return out;
    }
    ++p;
    while (p < end && *p != '"') {
      if (*p == '\\') {
        ++p;
        if (p >= end) break;
        switch (*p) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'u': p += 4; out += '?'; break;
          default: out += *p; break;
        }
        ++p;
      } else {
        out += *p++;
      }
    }
    if (p >= end) {
      ok = false;
      return out;
    }
    ++p;
    return out;
  }
  Json value(int depth = 0) {
    Json v;
    ws();
    if (p >= end || depth > 16) {
      ok = false;
      return v;
    }
    if (*p == '{') {
      v.kind = Json::Obj;
      ++p;
      ws();
      if (p < end && *p == '}') {
        ++p;
        return v;
      }
      while (ok) {
        ws();
        std::string k = string();
        ws();
        if (p >= end || *p != ':') {
          ok = false;
          break;
        }
        ++p;
        v.obj[k] = value(depth + 1);
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') {
          ++p;
          break;
        }
        ok = false;
      }
    } else if (*p == '[') {
      v.kind = Json::Arr;
      ++p;
      ws();
      if (p < end && *p == ']') {
        ++p;
        return v;
      }
      while (ok) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') {
          ++p;
          break;
        }
        ok = false;
      }
    } else if (*p == '"') {
      v.kind = Json::Str;
      v.str = string();
    } else if (lit("true")) {
      v.kind = Json::Bool;
      v.num = 1;
    } else if (lit("false")) {
      v.kind = Json::Bool;
    } else if (lit("null")) {
      v.kind = Json::Null;
    } else {
      char* e = nullptr;
      v.kind = Json::Num;
      v.num = std::strtod(p, &e);
      if (e == p) ok = false;
      p = e;
    }
    return v;
  }
};

// ------------------------------------------------------------- weights ----
const char* const kNames[kTensors] = {
#define ENC(l)                                                                                          \
  "encoder_layers." #l ".W1.weight", "encoder_layers." #l ".W1.bias", "encoder_layers." #l ".W2.weight", \
      "encoder_layers." #l ".W2.bias", "encoder_layers." #l ".W3.weight", "encoder_layers." #l ".W3.bias",  \
      "encoder_layers." #l ".W11.weight", "encoder_layers." #l ".W11.bias",                              \
      "encoder_layers." #l ".W12.weight", "encoder_layers." #l ".W12.bias",                              \
      "encoder_layers." #l ".W13.weight", "encoder_layers." #l ".W13.bias",                              \
      "encoder_layers." #l ".norm1.weight", "encoder_layers." #l ".norm1.bias",                          \
      "encoder_layers." #l ".norm2.weight", "encoder_layers." #l ".norm2.bias",                          \
      "encoder_layers." #l ".norm3.weight", "encoder_layers." #l ".norm3.bias",                          \
      "encoder_layers." #l ".dense.W_in.weight", "encoder_layers." #l ".dense.W_in.bias",                \
      "encoder_layers." #l ".dense.W_out.weight", "encoder_layers." #l ".dense.W_out.bias"
#define DEC(l)                                                                                          \
  "decoder_layers." #l ".W1.weight", "decoder_layers." #l ".W1.bias", "decoder_layers." #l ".W2.weight", \
      "decoder_layers." #l ".W2.bias", "decoder_layers." #l ".W3.weight", "decoder_layers." #l ".W3.bias",  \
      "decoder_layers." #l ".norm1.weight", "decoder_layers." #l ".norm1.bias",                          \
      "decoder_layers." #l ".norm2.weight", "decoder_layers." #l ".norm2.bias",                          \
      "decoder_layers." #l ".dense.W_in.weight", "decoder_layers." #l ".dense.W_in.bias",                \
      "decoder_layers." #l ".dense.W_out.weight", "decoder_layers." #l ".dense.W_out.bias"
    "features.embeddings.linear.weight",
    "features.embeddings.linear.bias",
    "features.edge_embedding.weight",
    "features.norm_edges.weight",
    "features.norm_edges.bias",
    "W_e.weight",
    "W_e.bias",
    "W_s.weight",
    ENC(0),
    ENC(1),
    ENC(2),
    DEC(0),
    DEC(1),
    DEC(2),
    "W_out.weight",
    "W_out.bias",
#undef ENC
#undef DEC
};

size_t expected_count(int i) {
  const std::string n = kNames[i];
  auto ends = [&](const char* s) {
    const size_t k = std::strlen(s);
    return n.size() >= k && n.compare(n.size() - k, k, s) == 0;
  };
  if (i == 0) return 16 * 66;
  if (i == 1) return 16;
  if (i == 2) return 128 * 416;
  if (i == 5) return 128 * 128;
  if (i == 7 || i == 116) return 21 * 128;
  if (i == 117) return 21;
  if (ends("W_in.weight") || ends("W_out.weight")) return 512 * 128;
  if (ends("W_in.bias")) return 512;
  if (n.rfind("encoder", 0) == 0 && (ends("W1.weight") || ends("W11.weight"))) return 128 * 384;
  if (n.rfind("decoder", 0) == 0 && ends("W1.weight")) return 128 * 512;
  if (ends(".weight") && (n.find(".W") != std::string::npos)) return 128 * 128;
  return 128;
}

struct HostArena {
  std::vector<float> data;
  size_t add(size_t n) {
    const size_t off = data.size();
    data.resize(off + ((n + 63) / 64) * 64, 0.0F);
    return off;
  }
};

// kpack16: rows [N][kin] (row-major), columns [c0, c0 + kd) -> [kd/16][N][16].
size_t pack_k16(HostArena& ar, const std::vector<const float*>& row_blocks, int rows_per_block, int kin, int c0,
                int kd) {
  const int N = static_cast<int>(row_blocks.size()) * rows_per_block;
  const size_t off = ar.add((size_t)N * kd);
  for (int n = 0; n < N; ++n) {
    const float* src = row_blocks[n / rows_per_block];
    const int rr = n % rows_per_block;
    for (int k = 0; k < kd; ++k) {
      const float v = src ? src[(size_t)rr * kin + c0 + k] : 0.0F;
      ar.data[off + ((size_t)(k / 16) * N + n) * 16 + (k % 16)] = v;
    }
  }
  return off;
}

// fp16 split of W [N][kin] (N outputs, kin inputs) for the fp16 MFMA:
// W = hi + lo / 2048 with hi = fp16(W) and lo = fp16((W - hi) * 2048), each
// stored as [kin / 8][N][8] halves (two per float slot). Returns the offset of
// hi; lo follows at hi + N * kin / 2.
size_t pack_f16_split(HostArena& ar, const float* W, int N, int kin) {
  const size_t half_slots = (size_t)N * kin / 2;
  const size_t off = ar.add(2 * half_slots);
  auto* hi = reinterpret_cast<_Float16*>(ar.data.data() + off);
  auto* lo = reinterpret_cast<_Float16*>(ar.data.data() + off + half_slots);
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < kin; ++k) {
      const float w = W[(size_t)n * kin + k];
      const _Float16 h = static_cast<_Float16>(w);
      const size_t at = ((size_t)(k / 8) * N + n) * 8 + k % 8;
      hi[at] = h;
      lo[at] = static_cast<_Float16>((w - static_cast<float>(h)) * 2048.0F);
    }
  return off;
}

// fp32 -> bf16, round to nearest even (NaN stays NaN).
uint16_t to_bf16(float f) {
  uint32_t u = 0;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// bf16 copy of n floats already packed at float offset src (same layout).
size_t copy_bf16(HostArena& ar, size_t src, size_t n) {
  const size_t off = ar.add((n + 1) / 2);
  auto* dst = reinterpret_cast<uint16_t*>(ar.data.data() + off);
  const float* s = ar.data.data() + src;
  for (size_t i = 0; i < n; ++i) dst[i] = to_bf16(s[i]);
  return off;
}

// fp16 copy of n floats already packed at float offset src (same layout).
size_t copy_f16(HostArena& ar, size_t src, size_t n) {
  const size_t off = ar.add((n + 1) / 2);
  auto* dst = reinterpret_cast<_Float16*>(ar.data.data() + off);
  const float* s = ar.data.data() + src;
  for (size_t i = 0; i < n; ++i) dst[i] = static_cast<_Float16>(s[i]);
  return off;
}

float from_bf16(uint16_t h) {
  const uint32_t u = static_cast<uint32_t>(h) << 16;
  float f = 0.0F;
  std::memcpy(&f, &u, 4);
  return f;
}

// The 16-bit forms of one weight: kHalfBf16 = bf16(w), kHalfBf16Lo = bf16(w - bf16(w))
// (the remainder of the split bf16 decode: w ~ hi + lo to about 16 significant bits,
// and hi + lo is exact in fp32), kHalfFp16 = fp16(w).
enum HalfForm { kHalfFp16 = 0, kHalfBf16 = 1, kHalfBf16Lo = 2 };
uint16_t to_half_form(float w, HalfForm form) {
  switch (form) {
    case kHalfBf16:
      return to_bf16(w);
    case kHalfBf16Lo:
      return to_bf16(w - from_bf16(to_bf16(w)));
    default:
      return __builtin_bit_cast(uint16_t, static_cast<_Float16>(w));
  }
}

// A 16-bit form of W [N][kin] as [kin / 8][N][8] (the B fragments of the 16x16x32 MFMA).
size_t pack_bf16_k8(HostArena& ar, const float* W, int N, int kin, HalfForm form = kHalfBf16) {
  const size_t off = ar.add((size_t)N * kin / 2);
  auto* dst = reinterpret_cast<uint16_t*>(ar.data.data() + off);
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < kin; ++k) dst[((size_t)(k / 8) * N + n) * 8 + k % 8] = to_half_form(W[(size_t)n * kin + k], form);
  return off;
}

// A 16-bit form of a t-layout matrix already packed at float offset src ([kin][ldo],
// inputs outer, the first N columns used) as [kin / 8][N][8]: the B fragments of the
// 16x16x32 MFMA, 8 consecutive inputs of one output per 16 bytes.
size_t pack_k8_t(HostArena& ar, size_t src, int kin, int N, int ldo, HalfForm form) {
  const size_t off = ar.add((size_t)N * kin / 2);
  auto* dst = reinterpret_cast<uint16_t*>(ar.data.data() + off);
  const float* s = ar.data.data() + src;
  for (int k = 0; k < kin; ++k)
    for (int n = 0; n < N; ++n) dst[((size_t)(k / 8) * N + n) * 8 + k % 8] = to_half_form(s[(size_t)k * ldo + n], form);
  return off;
}

// Transposed: W [N][kin] columns [c0, c0 + kd) -> [kd][ldo] (first N columns used).
size_t pack_t(HostArena& ar, const float* W, int N, int kin, int c0, int kd, int ldo) {
  const size_t off = ar.add((size_t)kd * ldo);
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < kd; ++k) ar.data[off + (size_t)k * ldo + n] = W[(size_t)n * kin + c0 + k];
  return off;
}

size_t copy_raw(HostArena& ar, const float* src, size_t n, size_t pad_to = 0) {
  const size_t off = ar.add(std::max(n, pad_to));
  std::memcpy(ar.data.data() + off, src, n * sizeof(float));
  return off;
}

// --------------------------------------------------------- workspace ----
struct DeviceArena {
  char* base = nullptr;
  size_t cap = 0;
  size_t used = 0;
  // busy: an event that follows every kernel still using the workspace (or
  // null); a workspace that has to grow is freed only after it.
  hipError_t reserve(size_t bytes, hipEvent_t busy) {
    if (bytes <= cap) return hipSuccess;
    if (busy) (void)hipEventSynchronize(busy);
    if (base) (void)hipFree(base);
    base = nullptr;
    cap = 0;
    hipError_t e = hipMalloc(&base, bytes);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // a failed allocation's error must not surface from a later launch check
      base = nullptr;
      return e;
    }
    cap = bytes;
    return hipSuccess;
  }
  void reset() { used = 0; }
  template <typename T>
  T* take(size_t n) {
    const size_t bytes = ((n * sizeof(T) + 255) / 256) * 256;
    T* p = reinterpret_cast<T*>(base + used);
    used += bytes;
    return p;
  }
};

template <typename T>
size_t aligned_bytes(size_t n) {
  return ((n * sizeof(T) + 255) / 256) * 256;
}

// ------------------------------------------------------- decode order ----
// cpp/modules/mpnn/decode_order_scalar.cpp:21-42,89-115
uint64_t splitmix64(uint64_t& state) {
  state += 0x9E3779B97F4A7C15ull;
  uint64_t z = state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

double uniform01(uint64_t& state) { return static_cast<double>(splitmix64(state) >> 11) * (1.0 / 9007199254740992.0); }

float normal_abs(uint64_t& state) {
  double u1 = uniform01(state);
  if (u1 <= 0.0) u1 = 1.0 / 9007199254740992.0;
  const double u2 = uniform01(state);
  const double radius = std::sqrt(-2.0 * std::log(u1));
  return static_cast<float>(std::fabs(radius * std::cos(6.283185307179586476925286766559 * u2)));
}

void random_order(const float* chain_mask, const float* residue_mask, int L, uint64_t seed, int32_t* order) {
  std::vector<float> scores(L);
  uint64_t state = seed;
  for (int r = 0; r < L; ++r) {
    const float c = chain_mask ? chain_mask[r] : 1.0F;
    const float mk = residue_mask ? residue_mask[r] : 1.0F;
    order[r] = r;
    scores[r] = (c * mk + 0.0001F) * normal_abs(state);
  }
  std::stable_sort(order, order + L, [&](int32_t l, int32_t r) {
    const float ls = scores[l], rs = scores[r];
    if (ls == rs) return l < r;
    return ls < rs;
  });
}

bool is_permutation(const int32_t* order, int L) {
  std::vector<unsigned char> seen(L, 0);
  for (int p = 0; p < L; ++p) {
    const int32_t r = order[p];
    if (r < 0 || r >= L || seen[r]) return false;
    seen[r] = 1;
  }
  return true;
}

void residue_mask_host(const uint8_t* src, int L, std::vector<float>& mask) {
  mask.assign(L, 0.0F);
  for (int r = 0; r < L; ++r) {
    const uint8_t* s = src + (size_t)r * 5;
    mask[r] = (s[0] && s[1] && s[2] && s[3]) ? 1.0F : 0.0F;
  }
}

}  // namespace

// Scratch of hkbs_pmpnn_design_device_noalloc: one static array per GPU that
// the library runs on (held until the process ends). Host code never uses the
// array's name as an address: hkbs_pmpnn_create looks up this device's
// address with hipGetSymbolAddress and keeps it in the context.
constexpr size_t kNoAllocScratchBytes = (size_t)128 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

struct hkbs_pmpnn {
  int device = 0;
  char* scratch = nullptr;      // this device's address of `scratch`
  hipStream_t stream = nullptr;
  hipStream_t side = nullptr;   // builds the decode schedule while the encoder runs
  hipEvent_t fork = nullptr;    // kNN graph ready (recorded on stream)
  hipEvent_t join = nullptr;    // schedule ready (recorded on side)
  hipEvent_t rows = nullptr;    // decode positions and the compact layer-0 table's row offsets ready (on side)
  float* weights = nullptr;
  ModelDev model{};
  DeviceArena arena;
  bool timing = false;
  bool timed = false;  // events hold a recorded design call
  hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
  uint32_t* fault = nullptr;  // device word raised by the last decode if a team barrier timed out
  DecodeArgs last_decode{};   // arguments of the last decode launch (for a one-workgroup rerun)
  int precision = HKBS_PRECISION_FP32;
  // Ragged scoring pipeline: chunk inputs go up on `side` and results come down on `down`, through two
  // staging slots of pinned host memory; per slot, events for inputs uploaded, chunk computed and results
  // copied down.
  hipStream_t down = nullptr;
  hipEvent_t score_ev[3][2] = {};
  char* pinned = nullptr;
  size_t pinned_cap = 0;
  // End of the last device entry point's work: those calls return while their
  // kernels may still run (on the caller's stream), and every later call on the
  // context waits for this event before it uses the workspace.
  hipEvent_t done = nullptr;
  bool done_recorded = false;
};

namespace {

hkbs_status hip_fail(hipError_t e, const char* what) {
  (void)e;
  return fail(HKBS_INTERNAL_ERROR, what);
}

#define HK_CHECK(expr, what)                      \
  do {                                            \
    hipError_t _e = (expr);                       \
    if (_e != hipSuccess) return hip_fail(_e, what); \
  } while (0)

// Calls on one context share its workspace. A device entry point returns while
// its kernels may still run on the caller's stream, so every call makes the
// stream it enqueues on wait, on the device, for the end of the previous device
// entry point's work before its first enqueue, and a device entry point records
// that end (ctx->done). A stream being captured into a HIP graph does neither:
// the caller orders the graph after earlier calls on the context.
hipEvent_t busy_event(const hkbs_pmpnn* ctx) { return ctx->done_recorded ? ctx->done : nullptr; }

hkbs_status after_previous_call(hkbs_pmpnn* ctx, hipStream_t s) {
  if (ctx->done_recorded) HK_CHECK(hipStreamWaitEvent(s, ctx->done, 0), "stream wait failed");
  return HKBS_OK;
}

hkbs_status record_call_end(hkbs_pmpnn* ctx, hipStream_t s) {
  HK_CHECK(hipEventRecord(ctx->done, s), "event record failed");
  ctx->done_recorded = true;
  return HKBS_OK;
}

hkbs_status build_model(hkbs_pmpnn* ctx, const float* const* t) {
  HostArena ar;
  struct Off {
    size_t pos_w, pos_b, edge_t, ne_g, ne_b, We_t, We_b, Ws;
    size_t W1b_dec_p, W1d_dec_p, Wlog_t, blog, Wlog_h, Wlog_f;
    size_t enc[kLayers][22];
    size_t dec[kLayers][24];
    size_t dec_h[kLayers][4];  // bf16 of W3_t, Win_t, Wout_t, W1da_t as MFMA B fragments (pack_k8_t)
    size_t dec_f[kLayers][4];  // fp16 of the same
    size_t dec_hl[kLayers][4];  // bf16 remainders of the same (split bf16 decode)
    size_t enc16[2 + 8 * kLayers];  // split-fp16 encoder weights: W_edge, W_e, then per layer
                                    // W1 W2 W3 W11 W12 W13 W_in W_out
  } o{};
  o.pos_w = copy_raw(ar, t[0], 16 * 66);
  o.pos_b = copy_raw(ar, t[1], 16);
  o.edge_t = pack_t(ar, t[2], 128, 416, 0, 416, 128);
  o.ne_g = copy_raw(ar, t[3], 128);
  o.ne_b = copy_raw(ar, t[4], 128);
  o.We_t = pack_t(ar, t[5], 128, 128, 0, 128, 128);
  o.We_b = copy_raw(ar, t[6], 128);
  o.Ws = copy_raw(ar, t[7], 21 * 128);
  for (int l = 0; l < kLayers; ++l) {
    const float* const* e = t + 8 + 22 * l;
    size_t* q = o.enc[l];
    q[0] = pack_t(ar, e[0], 128, 384, 0, 384, 128);   // W1_t
    q[1] = pack_t(ar, e[2], 128, 128, 0, 128, 128);   // W2_t
    q[2] = pack_t(ar, e[4], 128, 128, 0, 128, 128);   // W3_t
    q[3] = pack_t(ar, e[6], 128, 384, 0, 384, 128);   // W11_t
    q[4] = pack_t(ar, e[8], 128, 128, 0, 128, 128);   // W12_t
    q[5] = pack_t(ar, e[10], 128, 128, 0, 128, 128);  // W13_t
    q[6] = pack_t(ar, e[18], 512, 128, 0, 128, 512);  // Win_t
    q[7] = pack_t(ar, e[20], 128, 512, 0, 512, 128);  // Wout_t
    q[8] = copy_raw(ar, e[1], 128);                   // b1
    q[9] = copy_raw(ar, e[3], 128);                   // b2
    q[10] = copy_raw(ar, e[5], 128);                  // b3
    q[11] = copy_raw(ar, e[7], 128);                  // b11
    q[12] = copy_raw(ar, e[9], 128);                  // b12
    q[13] = copy_raw(ar, e[11], 128);                 // b13
    q[14] = copy_raw(ar, e[19], 512);                 // bin
    q[15] = copy_raw(ar, e[21], 128);                 // bout
    for (int i = 0; i < 6; ++i) q[16 + i] = copy_raw(ar, e[12 + i], 128);  // n1g n1b n2g n2b n3g n3b
  }
  {
    auto pk = [&](const float* W, int N, int kin) { return pack_f16_split(ar, W, N, kin); };
    size_t* q = o.enc16;
    q[0] = pk(t[2], 128, 416);  // W_edge
    q[1] = pk(t[5], 128, 128);  // W_e
    for (int l = 0; l < kLayers; ++l) {
      const float* const* e = t + 8 + 22 * l;
      size_t* ql = q + 2 + 8 * l;
      ql[0] = pk(e[0], 128, 384);   // W1
      ql[1] = pk(e[2], 128, 128);   // W2
      ql[2] = pk(e[4], 128, 128);   // W3
      ql[3] = pk(e[6], 128, 384);   // W11
      ql[4] = pk(e[8], 128, 128);   // W12
      ql[5] = pk(e[10], 128, 128);  // W13
      ql[6] = pk(e[18], 512, 128);  // W_in
      ql[7] = pk(e[20], 128, 512);  // W_out
    }
  }
  {
    std::vector<float> w1b(384 * 128), w1d(512 * 128);
    for (int l = 0; l < kLayers; ++l) {
      const float* W1 = t[74 + 14 * l];
      for (int n = 0; n < 128; ++n)
        for (int k = 0; k < 128; ++k) {
          w1b[(size_t)(l * 128 + n) * 128 + k] = W1[(size_t)n * 512 + 128 + k];
          w1d[(size_t)(l * 128 + n) * 128 + k] = W1[(size_t)n * 512 + 384 + k];
          if (l == 0) w1d[(size_t)(384 + n) * 128 + k] = W1[(size_t)n * 512 + k];
        }
    }
    o.W1b_dec_p = pack_k16(ar, {w1b.data()}, 384, 128, 0, 128);
    o.W1d_dec_p = pack_k16(ar, {w1d.data()}, 512, 128, 0, 128);
  }
  for (int l = 0; l < kLayers; ++l) {
    const float* const* d = t + 74 + 14 * l;
    size_t* q = o.dec[l];
    q[0] = pack_t(ar, d[0], 128, 512, 0, 128, 128);    // W1a_t
    q[1] = pack_k16(ar, {d[2]}, 128, 128, 0, 128);     // W2_p
    q[2] = pack_t(ar, d[4], 128, 128, 0, 128, 128);    // W3_t
    q[3] = pack_t(ar, d[10], 512, 128, 0, 128, 512);   // Win_t [128][512]
    q[4] = pack_t(ar, d[12], 128, 512, 0, 512, 128);   // Wout_t [512][128]
    {
      // [128][256]: columns 0..127 = W1d (inputs 384..511), 128..255 = W1a (inputs 0..127)
      const size_t off = ar.add(128 * 256);
      for (int n = 0; n < 128; ++n)
        for (int k = 0; k < 128; ++k) {
          ar.data[off + (size_t)k * 256 + n] = d[0][(size_t)n * 512 + 384 + k];
          ar.data[off + (size_t)k * 256 + 128 + n] = d[0][(size_t)n * 512 + k];
        }
      q[5] = off;
    }
    {
      // T[v][o] = sum_p W1c[o][p] W_s[v][p], in double then rounded.
      std::vector<float> T(21 * 128);
      for (int v = 0; v < 21; ++v)
        for (int oo = 0; oo < 128; ++oo) {
          double s = 0.0;
          for (int p = 0; p < 128; ++p) s += (double)d[0][(size_t)oo * 512 + 256 + p] * (double)t[7][(size_t)v * 128 + p];
          T[(size_t)v * 128 + oo] = static_cast<float>(s);
        }
      q[6] = copy_raw(ar, T.data(), T.size());
    }
    q[20] = pack_f16_split(ar, d[2], 128, 128);       // W2 hi, lo (fp16)
    {
      std::vector<float> w1b(128 * 128);  // W1b (inputs 128..255 of W1)
      for (int n = 0; n < 128; ++n)
        for (int k = 0; k < 128; ++k) w1b[(size_t)n * 128 + k] = d[0][(size_t)n * 512 + 128 + k];
      q[22] = pack_f16_split(ar, w1b.data(), 128, 128);  // W1b hi, lo (fp16)
    }
    q[21] = pack_bf16_k8(ar, d[2], 128, 128);         // W2 (bf16)
    q[23] = pack_bf16_k8(ar, d[2], 128, 128, kHalfBf16Lo);  // W2 bf16 remainder
    q[16] = pack_f16_split(ar, d[4], 128, 128);   // W3 hi, lo (fp16; teacher forcing)
    q[17] = pack_f16_split(ar, d[10], 512, 128);  // W_in
    q[18] = pack_f16_split(ar, d[12], 128, 512);  // W_out
    if (l + 1 < kLayers) {
      const float* Wn = t[74 + 14 * (l + 1)];
      std::vector<float> nx(256 * 128);
      for (int n = 0; n < 128; ++n)
        for (int k = 0; k < 128; ++k) {
          nx[(size_t)n * 128 + k] = Wn[(size_t)n * 512 + k];                // W1a of layer l+1
          nx[(size_t)(128 + n) * 128 + k] = Wn[(size_t)n * 512 + 384 + k];  // W1d of layer l+1
        }
      q[19] = pack_f16_split(ar, nx.data(), 256, 128);
    } else {
      q[19] = 0;
    }
    for (HalfForm form : {kHalfBf16, kHalfFp16, kHalfBf16Lo}) {
      size_t* dst = form == kHalfBf16 ? o.dec_h[l] : form == kHalfFp16 ? o.dec_f[l] : o.dec_hl[l];
      dst[0] = pack_k8_t(ar, q[2], 128, 128, 128, form);  // W3_t
      dst[1] = pack_k8_t(ar, q[3], 128, 512, 512, form);  // Win_t
      dst[2] = pack_k8_t(ar, q[4], 512, 128, 128, form);  // Wout_t
      dst[3] = pack_k8_t(ar, q[5], 128, 256, 256, form);  // W1da_t
    }
    q[7] = copy_raw(ar, d[1], 128);    // b1
    q[8] = copy_raw(ar, d[3], 128);    // b2
    q[9] = copy_raw(ar, d[5], 128);    // b3
    q[10] = copy_raw(ar, d[11], 512);  // bin
    q[11] = copy_raw(ar, d[13], 128);  // bout
    for (int i = 0; i < 4; ++i) q[12 + i] = copy_raw(ar, d[6 + i], 128);  // n1g n1b n2g n2b
  }
  o.Wlog_t = pack_t(ar, t[116], 21, 128, 0, 128, 32);
  o.blog = copy_raw(ar, t[117], 21, 32);
  o.Wlog_h = copy_bf16(ar, o.Wlog_t, 128 * 32);
  o.Wlog_f = copy_f16(ar, o.Wlog_t, 128 * 32);

  HK_CHECK(hipMalloc(&ctx->weights, ar.data.size() * sizeof(float)), "device allocation of weights failed");
  HK_CHECK(hipMemcpy(ctx->weights, ar.data.data(), ar.data.size() * sizeof(float), hipMemcpyHostToDevice),
           "weight upload failed");
  const float* B = ctx->weights;
  ModelDev& m = ctx->model;
  m.pos_w = B + o.pos_w;
  m.pos_b = B + o.pos_b;
  m.edge_t = B + o.edge_t;
  m.ne_g = B + o.ne_g;
  m.ne_b = B + o.ne_b;
  m.We_t = B + o.We_t;
  m.We_b = B + o.We_b;
  m.Ws = B + o.Ws;
  for (int l = 0; l < kLayers; ++l) {
    const size_t* q = o.enc[l];
    EncLayerDev& w = m.enc[l];
    w.W1_t = B + q[0];
    w.W2_t = B + q[1];
    w.W3_t = B + q[2];
    w.W11_t = B + q[3];
    w.W12_t = B + q[4];
    w.W13_t = B + q[5];
    w.Win_t = B + q[6];
    w.Wout_t = B + q[7];
    w.b1 = B + q[8];
    w.b2 = B + q[9];
    w.b3 = B + q[10];
    w.b11 = B + q[11];
    w.b12 = B + q[12];
    w.b13 = B + q[13];
    w.bin = B + q[14];
    w.bout = B + q[15];
    w.n1g = B + q[16];
    w.n1b = B + q[17];
    w.n2g = B + q[18];
    w.n2b = B + q[19];
    w.n3g = B + q[20];
    w.n3b = B + q[21];
  }
  for (int l = 0; l < kLayers; ++l) {
    const size_t* q = o.dec[l];
    DecLayerDev& w = m.dec[l];
    w.W1a_t = B + q[0];
    w.W2_p = B + q[1];
    w.W2h = B + q[20];
    w.W2l = B + q[20] + 128 * 128 / 2;
    w.W1b_s = reinterpret_cast<const uint16_t*>(B + q[22]);
    w.W2_b = reinterpret_cast<const uint16_t*>(B + q[21]);
    w.W3_h = reinterpret_cast<const uint16_t*>(B + o.dec_h[l][0]);
    w.Win_h = reinterpret_cast<const uint16_t*>(B + o.dec_h[l][1]);
    w.Wout_h = reinterpret_cast<const uint16_t*>(B + o.dec_h[l][2]);
    w.W1da_h = reinterpret_cast<const uint16_t*>(B + o.dec_h[l][3]);
    w.W3_f = reinterpret_cast<const uint16_t*>(B + o.dec_f[l][0]);
    w.Win_f = reinterpret_cast<const uint16_t*>(B + o.dec_f[l][1]);
    w.Wout_f = reinterpret_cast<const uint16_t*>(B + o.dec_f[l][2]);
    w.W1da_f = reinterpret_cast<const uint16_t*>(B + o.dec_f[l][3]);
    w.W2_bl = reinterpret_cast<const uint16_t*>(B + q[23]);
    w.W3_hl = reinterpret_cast<const uint16_t*>(B + o.dec_hl[l][0]);
    w.Win_hl = reinterpret_cast<const uint16_t*>(B + o.dec_hl[l][1]);
    w.Wout_hl = reinterpret_cast<const uint16_t*>(B + o.dec_hl[l][2]);
    w.W1da_hl = reinterpret_cast<const uint16_t*>(B + o.dec_hl[l][3]);
    w.W3_t = B + q[2];
    w.Win_t = B + q[3];
    w.Wout_t = B + q[4];
    w.W1da_t = B + q[5];
    w.T = B + q[6];
    w.b1 = B + q[7];
    w.b2 = B + q[8];
    w.b3 = B + q[9];
    w.bin = B + q[10];
    w.bout = B + q[11];
    w.n1g = B + q[12];
    w.n1b = B + q[13];
    w.n2g = B + q[14];
    w.n2b = B + q[15];
    w.W3_s = reinterpret_cast<const uint16_t*>(B + q[16]);
    w.Win_s = reinterpret_cast<const uint16_t*>(B + q[17]);
    w.Wout_s = reinterpret_cast<const uint16_t*>(B + q[18]);
    w.Wnext_s = (l + 1 < kLayers) ? reinterpret_cast<const uint16_t*>(B + q[19]) : nullptr;
  }
  m.W1b_dec_p = B + o.W1b_dec_p;
  m.W1d_dec_p = B + o.W1d_dec_p;
  m.Wlog_t = B + o.Wlog_t;
  m.blog = B + o.blog;
  m.Wlog_h = reinterpret_cast<const uint16_t*>(B + o.Wlog_h);
  m.Wlog_f = reinterpret_cast<const uint16_t*>(B + o.Wlog_f);
  {
    auto u16 = [&](size_t off) { return reinterpret_cast<const uint16_t*>(B + off); };
    const size_t* q = o.enc16;
    m.enc16.Wedge = u16(q[0]);
    m.enc16.We = u16(q[1]);
    for (int l = 0; l < kLayers; ++l) {
      const size_t* ql = q + 2 + 8 * l;
      Enc16LayerDev& w = m.enc16.layer[l];
      w.W1 = u16(ql[0]);
      w.W2 = u16(ql[1]);
      w.W3 = u16(ql[2]);
      w.W11 = u16(ql[3]);
      w.W12 = u16(ql[4]);
      w.W13 = u16(ql[5]);
      w.Win = u16(ql[6]);
      w.Wout = u16(ql[7]);
    }
  }
  return HKBS_OK;
}

// Device pointers of one request's encoder state.
struct EncodeBuffers {
  float* mask;
  float4* ca;
  int32_t* idx;
  float* d2;
  float* h_v;
  float* h_e;
  EncoderScratch scratch;
  float* msg_sum;  // [L][128] teacher-forced message sums
};

size_t encode_bytes(int L, int K) {
  const size_t S = (size_t)L * K;
  return aligned_bytes<float>(L) + aligned_bytes<float4>(L) + aligned_bytes<int32_t>(S) + aligned_bytes<float>(S) +
         aligned_bytes<float>((size_t)L * kH) + aligned_bytes<float>(S * kH) + aligned_bytes<float>((size_t)L * kPrefix) +
         aligned_bytes<float>(S * kH + L) + aligned_bytes<float>((size_t)L * kH);
}

EncodeBuffers take_encode(DeviceArena& ar, int L, int K) {
  const size_t S = (size_t)L * K;
  EncodeBuffers e{};
  e.mask = ar.take<float>(L);
  e.ca = ar.take<float4>(L);
  e.idx = ar.take<int32_t>(S);
  e.d2 = ar.take<float>(S);
  e.h_v = ar.take<float>((size_t)L * kH);
  e.h_e = ar.take<float>(S * kH);
  e.scratch.prefix = ar.take<float>((size_t)L * kPrefix);
  e.scratch.msg = ar.take<float>(S * kH + L);
  e.msg_sum = ar.take<float>((size_t)L * kH);
  return e;
}

// Featurisation and encoder: the reference's fp32 rounding sequence, or in the
// 16-bit modes the split-operand fp16 MFMA (fp32-level accuracy). In fp32 mode
// HKBS_ENCODER=mfma selects the MFMA encoder too (fp32-accurate, not the
// reference's rounding sequence).
bool mfma_encoder_forced() {
  const char* env = std::getenv("HKBS_ENCODER");
  return env && std::strcmp(env, "mfma") == 0;
}

hipError_t launch_featurise_encode(hkbs_pmpnn* ctx, const float* coords, const uint8_t* src, const int32_t* resid,
                                   const int32_t* chain, int L, int K, const EncodeBuffers& e) {
  if (ctx->precision != HKBS_PRECISION_FP32 || mfma_encoder_forced())
    return launch_encoder16(ctx->model, coords, src, resid, chain, e.idx, e.mask, L, K, e.h_v, e.h_e, e.scratch,
                            ctx->stream);
  hipError_t err = launch_edge_embed(ctx->model, coords, src, resid, chain, e.idx, L, K, e.h_e, ctx->stream);
  if (err != hipSuccess) return err;
  return launch_encoder(ctx->model, e.idx, e.mask, L, K, e.h_v, e.h_e, e.scratch, ctx->stream);
}

hipError_t run_encode(hkbs_pmpnn* ctx, const float* coords, const uint8_t* src, const int32_t* resid,
                      const int32_t* chain, int L, int K, const EncodeBuffers& e) {
  hipError_t err = launch_knn(coords, src, L, K, e.idx, e.d2, e.mask, e.ca, ctx->stream);
  if (err != hipSuccess) return err;
  return launch_featurise_encode(ctx, coords, src, resid, chain, L, K, e);
}

struct Inputs {
  float* coords;
  uint8_t* src;
  int32_t* resid;
  int32_t* chain;
  float* chain_mask;
  int32_t* true_tokens;
};

size_t input_bytes(int L) {
  return aligned_bytes<float>((size_t)L * 15) + aligned_bytes<uint8_t>((size_t)L * 5) + 2 * aligned_bytes<int32_t>(L) +
         aligned_bytes<float>(L) + aligned_bytes<int32_t>(L);
}

hkbs_status upload_inputs(hkbs_pmpnn* ctx, DeviceArena& ar, const float* coords, const uint8_t* src,
                          const int32_t* resid, const int32_t* chain, const float* chain_mask,
                          const int32_t* true_tokens, int L, Inputs& in) {
  in.coords = ar.take<float>((size_t)L * 15);
  in.src = ar.take<uint8_t>((size_t)L * 5);
  in.resid = ar.take<int32_t>(L);
  in.chain = ar.take<int32_t>(L);
  in.chain_mask = ar.take<float>(L);
  in.true_tokens = ar.take<int32_t>(L);
  hipStream_t s = ctx->stream;
  HK_CHECK(hipMemcpyAsync(in.coords, coords, (size_t)L * 15 * sizeof(float), hipMemcpyHostToDevice, s), "H2D failed");
  HK_CHECK(hipMemcpyAsync(in.src, src, (size_t)L * 5, hipMemcpyHostToDevice, s), "H2D failed");
  if (resid) HK_CHECK(hipMemcpyAsync(in.resid, resid, (size_t)L * 4, hipMemcpyHostToDevice, s), "H2D failed");
  else in.resid = nullptr;
  if (chain) HK_CHECK(hipMemcpyAsync(in.chain, chain, (size_t)L * 4, hipMemcpyHostToDevice, s), "H2D failed");
  else in.chain = nullptr;
  if (chain_mask) HK_CHECK(hipMemcpyAsync(in.chain_mask, chain_mask, (size_t)L * 4, hipMemcpyHostToDevice, s), "H2D failed");
  else in.chain_mask = nullptr;
  if (true_tokens) HK_CHECK(hipMemcpyAsync(in.true_tokens, true_tokens, (size_t)L * 4, hipMemcpyHostToDevice, s), "H2D failed");
  else in.true_tokens = nullptr;
  return HKBS_OK;
}

// Pass schedule of up to B orders: sched, pstart, npass, draw and scratch.
size_t schedule_bytes(int L, int K, int B) {
  const size_t nq = (size_t)B;
  return 2 * aligned_bytes<int32_t>(nq * L) + aligned_bytes<int32_t>(nq * (L + 2)) + aligned_bytes<int32_t>(nq) +
         aligned_bytes<int32_t>(sched_scratch_words(L, K, nq));
}

// The fp32 and split bf16 decodes read their layer-0 message rows from a table
// (launch_layer0_table, fp32-accurate) unless HKBS_DECODE_L0TABLE=off or the
// table would exceed kL0TableMaxBytes; in fp32 the results are the same either
// way, in split bf16 layer 0 is then fp32-accurate rather than split bf16.
constexpr size_t kL0TableMaxBytes = (size_t)4 << 30;
bool l0_table_wanted(int precision, int L) {
  if (precision != HKBS_PRECISION_FP32 && precision != HKBS_PRECISION_BF16X3) return false;
  if (const char* env = std::getenv("HKBS_DECODE_L0TABLE"); env && std::strcmp(env, "off") == 0) return false;
  const int K = std::min(kKmax, L);
  return l0_table_floats((size_t)L, (size_t)K) * sizeof(float) <= kL0TableMaxBytes;
}

size_t decode_bytes(int L, int K, int B, bool l0table) {
  const size_t S = (size_t)L * K;
  return aligned_bytes<float>(kLayers * S * kH) + aligned_bytes<float>((size_t)(kLayers + 1) * L * kH) +
         2 * aligned_bytes<int32_t>((size_t)B * L) + aligned_bytes<uint64_t>(B) +
         aligned_bytes<float>((size_t)B * kLayers * L * kH) + aligned_bytes<int32_t>((size_t)B * L) +
         aligned_bytes<float>((size_t)B * L * kV) + aligned_bytes<float>((size_t)B * L) + aligned_bytes<float>(B) +
         aligned_bytes<uint32_t>((size_t)B + 1) + 2 * aligned_bytes<int32_t>((size_t)B * L * K) +
         schedule_bytes(L, K, B) +
         (l0table ? aligned_bytes<float>(l0_table_floats(L, K)) + aligned_bytes<int32_t>((size_t)L + 1) : 0) +
         aligned_bytes<float4>((size_t)B * L * kRecFloat4);
}

hkbs_status enter(hkbs_pmpnn* ctx) {
  if (!ctx) return fail(HKBS_INVALID_ARGUMENT, "hkbs_pmpnn context is null");
  if (hipSetDevice(ctx->device) != hipSuccess) return fail(HKBS_UNAVAILABLE, "HIP device is not available");
  return HKBS_OK;
}

hkbs_status check_temperature(float temperature) {
  if (!std::isfinite(temperature) || temperature < 0.0F)
    return fail(HKBS_INVALID_ARGUMENT, "inverse-fold sampling_temp must be finite and >= 0");
  return HKBS_OK;
}

// Bytes a device design takes from its arena: the chosen-log-prob buffer of
// the device entry points, then design_on_device's buffers in its order.
size_t design_scratch_bytes(int L, int B, bool shared, bool l0table) {
  const int K = std::min(kKmax, L);
  const size_t S = (size_t)L * K, nq = shared ? 1 : (size_t)B;
  return aligned_bytes<float>((size_t)B * L) + encode_bytes(L, K) + aligned_bytes<float>(kLayers * S * kH) +
         aligned_bytes<float>((size_t)(kLayers + 1) * L * kH) + aligned_bytes<int32_t>((size_t)B * L) +
         aligned_bytes<float>((size_t)B * kLayers * L * kH) + aligned_bytes<uint32_t>((size_t)B + 1) +
         2 * aligned_bytes<int32_t>(nq * L * K) + aligned_bytes<int32_t>(nq * L) + aligned_bytes<int32_t>(nq * (L + 2)) +
         aligned_bytes<int32_t>(nq) + aligned_bytes<int32_t>(nq * L) + aligned_bytes<int32_t>(sched_scratch_words(L, K, nq)) +
         (l0table ? aligned_bytes<float>(l0_table_floats(L, K)) + aligned_bytes<int32_t>((size_t)L + 1) : 0) +
         aligned_bytes<float4>(nq * L * kRecFloat4);
}

// Reserves the context's workspace for need(l0table) bytes. The layer-0 table
// only saves time (the results are the same without it), so when that
// reservation fails the table is dropped (l0table = false) and the smaller
// reservation is tried before the call fails.
template <typename Need>
hkbs_status reserve_workspace(hkbs_pmpnn* ctx, const Need& need, bool& l0table) {
  DeviceArena& ar = ctx->arena;
  if (ar.reserve(need(l0table), busy_event(ctx)) == hipSuccess) return HKBS_OK;
  if (l0table) {
    l0table = false;
    if (ar.reserve(need(false), busy_event(ctx)) == hipSuccess) return HKBS_OK;
  }
  return fail(HKBS_INTERNAL_ERROR, "device workspace allocation failed");
}

// A device entry point runs its work on the caller's stream (the context's own
// when none is given). *capturing tells whether that stream is being captured
// into a HIP graph: a captured call neither waits for nor records the end of
// other calls (after_previous_call, record_call_end).
hkbs_status adopt_caller_stream(hkbs_pmpnn* ctx, void* stream, bool* capturing) {
  if (stream) ctx->stream = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HK_CHECK(hipStreamIsCapturing(ctx->stream, &cs), "stream capture query failed");
  *capturing = cs != hipStreamCaptureStatusNone;
  return HKBS_OK;
}

// Shared implementation of the device design path. All pointers device.
hkbs_status design_on_device(hkbs_pmpnn* ctx, const float* coords, const uint8_t* src, const int32_t* resid,
                             const int32_t* chain, const float* chain_mask, const int32_t* true_tokens, int L, int B,
                             const int32_t* orders, int shared, const uint64_t* seeds, float temperature, int greedy,
                             int32_t* tokens, float* log_probs, float* scores, DeviceArena& ar, float* chosen,
                             bool l0table) {
  // The decode runs as an ordinary launch whose grid is resident at once, with
  // bounded team barriers; a cooperative launch is not offered.
  if (const char* mode = std::getenv("HKBS_DECODE_LAUNCH"); mode && std::strcmp(mode, "cooperative") == 0)
    return fail(HKBS_UNIMPLEMENTED, "cooperative decode launch is not supported");
  const int K = std::min(kKmax, L);
  const size_t S = (size_t)L * K;
  EncodeBuffers e = take_encode(ar, L, K);
  float* E1 = ar.take<float>(kLayers * S * kH);
  float* Q = ar.take<float>((size_t)(kLayers + 1) * L * kH);
  int32_t* pos = ar.take<int32_t>((size_t)B * L);
  float* R = ar.take<float>((size_t)B * kLayers * L * kH);
  uint32_t* sync = ar.take<uint32_t>((size_t)B + 1);  // B team counters + fault word
  const size_t nq = shared ? 1 : (size_t)B;
  int32_t* nbj = ar.take<int32_t>(nq * L * K);
  int32_t* nbp = ar.take<int32_t>(nq * L * K);
  int32_t* sched = ar.take<int32_t>(nq * L);
  int32_t* pstart = ar.take<int32_t>(nq * (L + 2));
  int32_t* npass = ar.take<int32_t>(nq);
  int32_t* draw = ar.take<int32_t>(nq * L);
  int32_t* sched_tmp = ar.take<int32_t>(sched_scratch_words(L, K, nq));
  float* l0tab = l0table ? ar.take<float>(l0_table_floats(L, K)) : nullptr;
  // one shared order: the compact table (rows a slot can use in that order)
  int32_t* l0base = l0table && shared ? ar.take<int32_t>((size_t)L + 1) : nullptr;
  float4* rec = ar.take<float4>(nq * L * kRecFloat4);
  if (ar.used > ar.cap) return fail(HKBS_INTERNAL_ERROR, "design workspace exceeds its reservation");
  ctx->fault = sync + B;
  DecodeArgs a{};
  a.idx = e.idx;
  a.mask = e.mask;
  a.h_v = e.h_v;
  a.E1 = E1;
  a.Q = Q;
  a.orders = orders;
  a.shared_order = shared;
  a.pos = pos;
  a.chain_mask = chain_mask;
  a.true_tokens = true_tokens;
  a.seeds = seeds;
  a.temperature = temperature;
  a.greedy = greedy || temperature <= 0.0F;
  a.L = L;
  a.K = K;
  a.B = B;
  a.R = R;
  a.tokens = tokens;
  a.log_probs = log_probs;
  a.scores = scores;
  a.chosen_lp = chosen;
  a.sync = sync;
  a.fault = sync + B;
  a.nbj = nbj;
  a.nbp = nbp;
  a.sched = sched;
  a.pstart = pstart;
  a.npass = npass;
  a.draw = draw;
  a.sched_tmp = sched_tmp;
  a.precision = ctx->precision;
  a.l0tab = l0tab;
  a.l0base = l0base;
  a.rec = rec;
  if (a.precision == HKBS_PRECISION_BF16 || a.precision == HKBS_PRECISION_FP16) {
    // bf16 and fp16 modes read the message rows' inputs in fp16: E1 and the Q blocks 0..2 share E1's space
    // (3 S + 3 L halves <= 3 S floats), R rows take half of R's.
    _Float16* E1h = reinterpret_cast<_Float16*>(E1);
    a.E1h = E1h;
    a.Qh = E1h + (size_t)kLayers * S * kH;
    a.Rh = reinterpret_cast<_Float16*>(R);
    a.E1 = nullptr;
  }
  const int team = decode_team_size(a.precision, B, 8);
  a.max_members = decode_group(a.precision, team) * team;
  a.pass_granule = team;
  if (const char* env = std::getenv("HKBS_DECODE_MAX_MEMBERS"))
    a.max_members = std::max(1, std::min(a.max_members, std::atoi(env)));
  ctx->last_decode = a;
  // The decode schedule needs only the kNN graph and the orders: it is built
  // on the side stream while the encoder runs, and the decode waits for it.
  // The encoder is enqueued first so that its launches do not queue behind
  // the schedule's on the host.
  if (ctx->timing) HK_CHECK(hipEventRecord(ctx->ev[0], ctx->stream), "event record failed");
  HK_CHECK(launch_knn(coords, src, L, K, e.idx, e.d2, e.mask, e.ca, ctx->stream), "kNN launch failed");
  HK_CHECK(hipEventRecord(ctx->fork, ctx->stream), "event record failed");
  HK_CHECK(launch_featurise_encode(ctx, coords, src, resid, chain, L, K, e), "encoder launch failed");
  HK_CHECK(hipStreamWaitEvent(ctx->side, ctx->fork, 0), "stream wait failed");
  HK_CHECK(launch_positions(orders, L, shared ? 1 : B, shared, pos, ctx->side), "position kernel failed");
  if (l0base) HK_CHECK(launch_l0_rows(e.idx, pos, L, K, l0base, ctx->side), "layer-0 table rows failed");
  HK_CHECK(hipEventRecord(ctx->rows, ctx->side), "event record failed");
  HK_CHECK(launch_decode_schedule(a, ctx->side), "decode schedule launch failed");
  HK_CHECK(hipEventRecord(ctx->join, ctx->side), "event record failed");
  if (ctx->timing) HK_CHECK(hipEventRecord(ctx->ev[1], ctx->stream), "event record failed");
  HK_CHECK(launch_decoder_precompute(ctx->model, e.h_v, e.h_e, L, K, E1, Q, ctx->stream, const_cast<_Float16*>(a.E1h),
                                     const_cast<_Float16*>(a.Qh)),
           "decoder precompute failed");
  HK_CHECK(launch_zero(reinterpret_cast<float*>(sync), (size_t)B + 1, ctx->stream), "workspace clear failed");
  // The table needs the positions and its row offsets; it is built while the
  // schedule (a few workgroups on the side stream) may still run.
  HK_CHECK(hipStreamWaitEvent(ctx->stream, ctx->rows, 0), "stream wait failed");
  if (l0tab)
    HK_CHECK(launch_layer0_table(ctx->model, E1, Q, e.idx, pos, l0base, L, K, l0tab, ctx->stream), "layer-0 table failed");
  HK_CHECK(hipStreamWaitEvent(ctx->stream, ctx->join, 0), "stream wait failed");  // the schedule
  HK_CHECK(launch_step_records(ctx->model, a, rec, ctx->stream), "step records launch failed");
  if (ctx->timing) HK_CHECK(hipEventRecord(ctx->ev[2], ctx->stream), "event record failed");
  HK_CHECK(launch_decode(ctx->model, a, ctx->stream, team), "decode launch failed");
  if (ctx->timing) {
    HK_CHECK(hipEventRecord(ctx->ev[3], ctx->stream), "event record failed");
    ctx->timed = true;
  }
  return HKBS_OK;
}

}  // namespace

hkbs_status hkbs::report_error(hkbs_status code, const char* detail) { return fail(code, detail); }

extern "C" {

const char* hkbs_last_error(void) { return g_last_error; }

const char* hkbs_version(void) { return "hikoboshi-amd 0.1.0 (gfx950, ProteinMPNN v_48_020)"; }

int32_t hkbs_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

hkbs_status hkbs_pmpnn_create(const uint8_t* data, size_t nbytes, int32_t device, hkbs_pmpnn** out) {
  if (!out) return fail(HKBS_INVALID_ARGUMENT, "output context pointer is null");
  *out = nullptr;
  if (!data || nbytes < 8) return fail(HKBS_INVALID_ARGUMENT, "weight package is empty");
  uint64_t hlen = 0;
  std::memcpy(&hlen, data, 8);
  if (hlen > nbytes - 8) return fail(HKBS_INVALID_ARGUMENT, "safetensors header length exceeds the package");
  JsonParser jp{reinterpret_cast<const char*>(data) + 8, reinterpret_cast<const char*>(data) + 8 + hlen};
  Json header = jp.value();
  if (!jp.ok || header.kind != Json::Obj) return fail(HKBS_INVALID_ARGUMENT, "safetensors header is not valid JSON");
  const size_t base = 8 + hlen;
  std::vector<std::vector<float>> storage(kTensors);
  std::vector<const float*> ptrs(kTensors);
  for (int i = 0; i < kTensors; ++i) {
    auto it = header.obj.find(kNames[i]);
    if (it == header.obj.end()) return fail(HKBS_INVALID_ARGUMENT, "weight package is missing a v_48_020 tensor");
    const Json& t = it->second;
    auto dt = t.obj.find("dtype");
    auto offs = t.obj.find("data_offsets");
    if (dt == t.obj.end() || dt->second.str != "F32" || offs == t.obj.end() || offs->second.arr.size() != 2)
      return fail(HKBS_INVALID_ARGUMENT, "weight package tensor is not F32 with data offsets");
    const size_t s = static_cast<size_t>(offs->second.arr[0].num);
    const size_t e = static_cast<size_t>(offs->second.arr[1].num);
    const size_t count = expected_count(i);
    if (e < s || e - s != count * 4 || base + e > nbytes)
      return fail(HKBS_INVALID_ARGUMENT, "weight package tensor has the wrong size for v_48_020");
    storage[i].resize(count);
    std::memcpy(storage[i].data(), data + base + s, count * 4);
    ptrs[i] = storage[i].data();
  }
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(HKBS_UNAVAILABLE, "no HIP device is available");
  if (device < 0 || device >= ndev) return fail(HKBS_INVALID_ARGUMENT, "HIP device index is out of range");
  if (hipSetDevice(device) != hipSuccess) return fail(HKBS_UNAVAILABLE, "HIP device is not available");
  hkbs_pmpnn* ctx = new hkbs_pmpnn();
  ctx->device = device;
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&ctx->side, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->fork, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->join, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->rows, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->done, hipEventDisableTiming) != hipSuccess) {
    hkbs_pmpnn_destroy(ctx);
    return fail(HKBS_UNAVAILABLE, "HIP stream creation failed");
  }
  void* sp = nullptr;
  if (hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)) != hipSuccess || !sp) {
    hkbs_pmpnn_destroy(ctx);
    return fail(HKBS_UNAVAILABLE, "device scratch of the allocation-free design is not available");
  }
  ctx->scratch = static_cast<char*>(sp);
  const hkbs_status st = build_model(ctx, ptrs.data());
  if (st != HKBS_OK) {
    hkbs_pmpnn_destroy(ctx);
    return st;
  }
  *out = ctx;
  return HKBS_OK;
}

void hkbs_pmpnn_destroy(hkbs_pmpnn* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  if (ctx->side) (void)hipStreamSynchronize(ctx->side);
  if (ctx->down) (void)hipStreamSynchronize(ctx->down);
  // a device entry point's kernels may still run on the caller's stream
  if (ctx->done_recorded) (void)hipEventSynchronize(ctx->done);
  for (hipEvent_t& ev : ctx->ev)
    if (ev) (void)hipEventDestroy(ev);
  for (auto& evs : ctx->score_ev)
    for (hipEvent_t& ev : evs)
      if (ev) (void)hipEventDestroy(ev);
  if (ctx->pinned) (void)hipHostFree(ctx->pinned);
  if (ctx->down) (void)hipStreamDestroy(ctx->down);
  if (ctx->fork) (void)hipEventDestroy(ctx->fork);
  if (ctx->join) (void)hipEventDestroy(ctx->join);
  if (ctx->rows) (void)hipEventDestroy(ctx->rows);
  if (ctx->done) (void)hipEventDestroy(ctx->done);
  if (ctx->side) (void)hipStreamDestroy(ctx->side);
  if (ctx->arena.base) (void)hipFree(ctx->arena.base);
  if (ctx->weights) (void)hipFree(ctx->weights);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

hkbs_status hkbs_pmpnn_decode_order(const float* chain_mask, const uint8_t* atom_sources, int32_t L, uint64_t seed,
                                    int32_t* order) {
  if (L < 0) return fail(HKBS_INVALID_ARGUMENT, "residue count is negative");
  if (L > 0 && (!atom_sources || !order)) return fail(HKBS_INVALID_ARGUMENT, "decode order pointers must be non-null");
  std::vector<float> mask;
  residue_mask_host(atom_sources, L, mask);
  random_order(chain_mask, mask.data(), L, seed, order);
  return HKBS_OK;
}

hkbs_status hkbs_pmpnn_backbone_noise(const float* coords, const uint8_t* atom_sources, int32_t L, float sigma,
                                      uint64_t seed, float* out) {
  if (L < 0) return fail(HKBS_INVALID_ARGUMENT, "residue count is negative");
  if (!std::isfinite(sigma) || sigma < 0.0F) return fail(HKBS_INVALID_ARGUMENT, "inverse-fold backbone_noise must be finite and >= 0");
  if (L > 0 && (!coords || !atom_sources || !out)) return fail(HKBS_INVALID_ARGUMENT, "backbone noise pointers must be non-null");
  if (L > 0) backbone_noise_host(coords, atom_sources, L, sigma, seed, out);
  return HKBS_OK;
}

hkbs_status hkbs_pmpnn_design(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                              const int32_t* residue_indices, const int32_t* chain_labels, const float* chain_mask,
                              const int32_t* true_tokens, int32_t L, int32_t B, int32_t order_mode,
                              const int32_t* orders, const uint64_t* order_seeds, const uint64_t* sampler_seeds,
                              float temperature, int32_t greedy, int32_t* tokens, float* log_probs,
                              int32_t* orders_out, float* scores) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (L < 0) return fail(HKBS_INVALID_ARGUMENT, "residue count is negative");
  if (B <= 0) return fail(HKBS_INVALID_ARGUMENT, "inverse-fold num_seqs must be greater than zero");
  if ((st = check_temperature(temperature)) != HKBS_OK) return st;
  if (L == 0) return HKBS_OK;
  if (!coords || !atom_sources) return fail(HKBS_INVALID_ARGUMENT, "inverse-fold structure must provide canonical backbone atoms");
  if (!sampler_seeds || !tokens) return fail(HKBS_INVALID_ARGUMENT, "sampler seeds and token output must be non-null");

  // Decoding orders on the host (bit-exact reference routine).
  int shared = 0;
  std::vector<int32_t> host_orders;
  std::vector<float> rmask;
  residue_mask_host(atom_sources, L, rmask);
  switch (order_mode) {
    case HKBS_ORDER_RANDOM:
      if (!order_seeds) return fail(HKBS_INVALID_ARGUMENT, "random decode order needs order seeds");
      host_orders.resize((size_t)B * L);
      for (int b = 0; b < B; ++b) random_order(chain_mask, rmask.data(), L, order_seeds[b], host_orders.data() + (size_t)b * L);
      break;
    case HKBS_ORDER_INPUT_PER_SEQUENCE:
      if (!orders) return fail(HKBS_INVALID_ARGUMENT, "input decode orders are null");
      host_orders.assign(orders, orders + (size_t)B * L);
      for (int b = 0; b < B; ++b)
        if (!is_permutation(orders + (size_t)b * L, L))
          return fail(HKBS_INVALID_ARGUMENT, "ProteinMPNN input decoding_order must be a permutation");
      break;
    case HKBS_ORDER_INPUT_SHARED:
      if (!orders) return fail(HKBS_INVALID_ARGUMENT, "input decode order is null");
      if (!is_permutation(orders, L)) return fail(HKBS_INVALID_ARGUMENT, "ProteinMPNN input decoding_order must be a permutation");
      host_orders.assign(orders, orders + L);
      shared = 1;
      break;
    case HKBS_ORDER_N_TO_C:
      host_orders.resize(L);
      std::iota(host_orders.begin(), host_orders.end(), 0);
      shared = 1;
      break;
    default:
      return fail(HKBS_INVALID_ARGUMENT, "unknown decode order mode");
  }

  const int K = std::min(kKmax, L);
  const size_t norders = shared ? (size_t)L : (size_t)B * L;
  bool l0table = l0_table_wanted(ctx->precision, L);
  const auto need = [&](bool tab) {
    return input_bytes(L) + encode_bytes(L, K) + decode_bytes(L, K, B, tab) + aligned_bytes<int32_t>(norders) +
           aligned_bytes<uint64_t>(B) + aligned_bytes<int32_t>((size_t)B * L) + aligned_bytes<float>((size_t)B * L * kV) +
           aligned_bytes<float>(B) + aligned_bytes<float>((size_t)B * L) + (64u << 10);
  };
  DeviceArena& ar = ctx->arena;
  if ((st = reserve_workspace(ctx, need, l0table)) != HKBS_OK) return st;
  if ((st = after_previous_call(ctx, ctx->stream)) != HKBS_OK) return st;
  ar.reset();
  Inputs in{};
  if ((st = upload_inputs(ctx, ar, coords, atom_sources, residue_indices, chain_labels, chain_mask, true_tokens, L, in)) != HKBS_OK)
    return st;
  int32_t* d_orders = ar.take<int32_t>(norders);
  uint64_t* d_seeds = ar.take<uint64_t>(B);
  int32_t* d_tokens = ar.take<int32_t>((size_t)B * L);
  float* d_lp = ar.take<float>((size_t)B * L * kV);
  float* d_scores = ar.take<float>(B);
  float* d_chosen = ar.take<float>((size_t)B * L);
  hipStream_t s = ctx->stream;
  HK_CHECK(hipMemcpyAsync(d_orders, host_orders.data(), norders * 4, hipMemcpyHostToDevice, s), "H2D failed");
  HK_CHECK(hipMemcpyAsync(d_seeds, sampler_seeds, (size_t)B * 8, hipMemcpyHostToDevice, s), "H2D failed");
  if ((st = design_on_device(ctx, in.coords, in.src, in.resid, in.chain, in.chain_mask, in.true_tokens, L, B, d_orders,
                             shared, d_seeds, temperature, greedy, d_tokens, log_probs ? d_lp : nullptr,
                             d_scores, ar, d_chosen, l0table)) != HKBS_OK)
    return st;
  HK_CHECK(hipMemcpyAsync(tokens, d_tokens, (size_t)B * L * 4, hipMemcpyDeviceToHost, s), "D2H failed");
  if (log_probs) HK_CHECK(hipMemcpyAsync(log_probs, d_lp, (size_t)B * L * kV * 4, hipMemcpyDeviceToHost, s), "D2H failed");
  if (scores) HK_CHECK(hipMemcpyAsync(scores, d_scores, (size_t)B * 4, hipMemcpyDeviceToHost, s), "D2H failed");
  uint32_t fault = 0;
  HK_CHECK(hipMemcpyAsync(&fault, ctx->fault, sizeof(fault), hipMemcpyDeviceToHost, s), "D2H failed");
  HK_CHECK(hipStreamSynchronize(s), "design kernels failed");
  if (fault) {
    // A team of workgroups could not run together (the device was busy with
    // other work): decode again with one workgroup per sequence.
    DecodeArgs one = ctx->last_decode;
    one.max_members = decode_group(one.precision, 1);  // steps one workgroup can hold
    one.pass_granule = 1;
    HK_CHECK(launch_decode_schedule(one, s), "decode schedule launch failed");
    HK_CHECK(launch_step_records(ctx->model, one, const_cast<float4*>(one.rec), s), "step records launch failed");
    HK_CHECK(launch_decode(ctx->model, one, s, 1), "decode launch failed");
    HK_CHECK(hipMemcpyAsync(tokens, d_tokens, (size_t)B * L * 4, hipMemcpyDeviceToHost, s), "D2H failed");
    if (log_probs) HK_CHECK(hipMemcpyAsync(log_probs, d_lp, (size_t)B * L * kV * 4, hipMemcpyDeviceToHost, s), "D2H failed");
    if (scores) HK_CHECK(hipMemcpyAsync(scores, d_scores, (size_t)B * 4, hipMemcpyDeviceToHost, s), "D2H failed");
    HK_CHECK(hipStreamSynchronize(s), "design kernels failed");
  }
  if (orders_out) {
    for (int b = 0; b < B; ++b)
      std::memcpy(orders_out + (size_t)b * L, host_orders.data() + (shared ? 0 : (size_t)b * L), (size_t)L * 4);
  }
  return HKBS_OK;
}

hkbs_status hkbs_pmpnn_design_device(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                                     const int32_t* residue_indices, const int32_t* chain_labels, const float* chain_mask,
                                     const int32_t* true_tokens, int32_t L, int32_t B, const int32_t* orders,
                                     int32_t shared_order, const uint64_t* sampler_seeds, float temperature,
                                     int32_t greedy, int32_t* tokens, float* log_probs, float* scores, void* stream) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (L < 0) return fail(HKBS_INVALID_ARGUMENT, "residue count is negative");
  if (B <= 0) return fail(HKBS_INVALID_ARGUMENT, "inverse-fold num_seqs must be greater than zero");
  if ((st = check_temperature(temperature)) != HKBS_OK) return st;
  if (L == 0) return HKBS_OK;
  if (!coords || !atom_sources || !orders || !sampler_seeds || !tokens)
    return fail(HKBS_INVALID_ARGUMENT, "device design pointers must be non-null");
  const int K = std::min(kKmax, L);
  bool l0table = l0_table_wanted(ctx->precision, L);
  const auto need = [&](bool tab) {
    return encode_bytes(L, K) + decode_bytes(L, K, B, tab) + aligned_bytes<float>((size_t)B * L) + (64u << 10);
  };
  DeviceArena& ar = ctx->arena;
  hipStream_t saved = ctx->stream;
  bool capturing = false;
  if ((st = adopt_caller_stream(ctx, stream, &capturing)) != HKBS_OK ||
      (st = reserve_workspace(ctx, need, l0table)) != HKBS_OK ||
      (!capturing && (st = after_previous_call(ctx, ctx->stream)) != HKBS_OK)) {
    ctx->stream = saved;
    return st;
  }
  ar.reset();
  float* chosen = ar.take<float>((size_t)B * L);
  st = design_on_device(ctx, coords, atom_sources, residue_indices, chain_labels, chain_mask, true_tokens, L, B, orders,
                        shared_order != 0, sampler_seeds, temperature, greedy, tokens, log_probs, scores, ar, chosen,
                        l0table);
  if (!capturing) {  // recorded also after a failure: part of the work may have been enqueued
    const hkbs_status end = record_call_end(ctx, ctx->stream);
    if (st == HKBS_OK) st = end;
  }
  ctx->stream = saved;
  return st;
}

hkbs_status hkbs_pmpnn_design_device_noalloc(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                                             const int32_t* residue_indices, const int32_t* chain_labels,
                                             const float* chain_mask, const int32_t* true_tokens, int32_t L, int32_t B,
                                             const int32_t* orders, int32_t shared_order,
                                             const uint64_t* sampler_seeds, float temperature, int32_t greedy,
                                             int32_t* tokens, float* log_probs, float* scores, void* stream) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (L < 0) return fail(HKBS_INVALID_ARGUMENT, "residue count is negative");
  if (B <= 0) return fail(HKBS_INVALID_ARGUMENT, "inverse-fold num_seqs must be greater than zero");
  if ((st = check_temperature(temperature)) != HKBS_OK) return st;
  if (L == 0) return HKBS_OK;
  if (!coords || !atom_sources || !orders || !sampler_seeds || !tokens)
    return fail(HKBS_INVALID_ARGUMENT, "device design pointers must be non-null");
  // The layer-0 table is used when it fits beside the rest (same results without it).
  bool l0table = l0_table_wanted(ctx->precision, L);
  if (l0table && design_scratch_bytes(L, B, shared_order != 0, true) > kNoAllocScratchBytes) l0table = false;
  if (design_scratch_bytes(L, B, shared_order != 0, l0table) > kNoAllocScratchBytes)
    return fail(HKBS_INVALID_ARGUMENT,
                "request needs more device scratch than the allocation-free design holds (128 MiB)");
  DeviceArena ar;  // borrows this device's static scratch; never freed
  ar.base = ctx->scratch;
  ar.cap = kNoAllocScratchBytes;
  hipStream_t saved = ctx->stream;
  bool capturing = false;
  if ((st = adopt_caller_stream(ctx, stream, &capturing)) != HKBS_OK ||
      (!capturing && (st = after_previous_call(ctx, ctx->stream)) != HKBS_OK)) {
    ctx->stream = saved;
    return st;
  }
  float* chosen = ar.take<float>((size_t)B * L);
  st = design_on_device(ctx, coords, atom_sources, residue_indices, chain_labels, chain_mask, true_tokens, L, B, orders,
                        shared_order != 0, sampler_seeds, temperature, greedy, tokens, log_probs, scores, ar, chosen,
                        l0table);
  if (!capturing) {
    const hkbs_status end = record_call_end(ctx, ctx->stream);
    if (st == HKBS_OK) st = end;
  }
  ctx->stream = saved;
  return st;
}

hkbs_status hkbs_pmpnn_set_precision(hkbs_pmpnn* ctx, int32_t precision) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (precision != HKBS_PRECISION_FP32 && precision != HKBS_PRECISION_BF16 && precision != HKBS_PRECISION_FP16 &&
      precision != HKBS_PRECISION_BF16X3)
    return fail(HKBS_INVALID_ARGUMENT, "unknown precision");
  ctx->precision = precision;
  return HKBS_OK;
}

hkbs_status hkbs_pmpnn_set_timing(hkbs_pmpnn* ctx, int32_t enable) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (enable && !ctx->ev[0])
    for (hipEvent_t& ev : ctx->ev)
      if (hipEventCreate(&ev) != hipSuccess) return fail(HKBS_INTERNAL_ERROR, "HIP event creation failed");
  ctx->timing = enable != 0;
  ctx->timed = false;
  return HKBS_OK;
}

hkbs_status hkbs_pmpnn_last_timing(hkbs_pmpnn* ctx, float* ms) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (!ms) return fail(HKBS_INVALID_ARGUMENT, "timing output is null");
  if (!ctx->timed) return fail(HKBS_FAILED_PRECONDITION, "no timed design call has been recorded");
  HK_CHECK(hipEventSynchronize(ctx->ev[3]), "event synchronisation failed");
  for (int i = 0; i < 3; ++i) HK_CHECK(hipEventElapsedTime(&ms[i], ctx->ev[i], ctx->ev[i + 1]), "event timing failed");
  return HKBS_OK;
}

}  // extern "C"

namespace {

// One teacher-forced pass over n_res residues (one protein, or a ragged
// chunk of proteins with the same K). All pointers are device memory except
// where noted; seg/offsets describe the chunk for the kNN (null = one protein).
hkbs_status teacher_forced_chunk(hkbs_pmpnn* ctx, const float* coords, const uint8_t* src, const int32_t* resid,
                                 const int32_t* chain, const int32_t* tokens, const int32_t* pos, int L, int K,
                                 const int32_t* seg, const int64_t* offsets, float* log_probs, DeviceArena& ar) {
  EncodeBuffers e = take_encode(ar, L, K);
  float* Q = ar.take<float>((size_t)(kLayers + 1) * L * kH);
  float* NB = ar.take<float>((size_t)L * 256);
  hipStream_t s = ctx->stream;
  HK_CHECK(launch_knn(coords, src, L, K, e.idx, e.d2, e.mask, e.ca, s, seg, offsets), "kNN launch failed");
  // Teacher-forced log-probs are not temperature-scaled, so the 1e-4 bar leaves room for the fp32-accurate
  // split-operand MFMA encoder (about 2x the throughput of the reference-order encoder).
  HK_CHECK(launch_encoder16(ctx->model, coords, src, resid, chain, e.idx, e.mask, L, K, e.h_v, e.h_e, e.scratch, s),
           "encoder launch failed");
  HK_CHECK(launch_q_precompute(ctx->model, e.h_v, L, Q, s), "decoder precompute failed");
  TfArgs a{};
  a.idx = e.idx;
  a.pos = pos;
  a.mask = e.mask;
  a.tokens = tokens;
  a.h_e = e.h_e;
  a.Q = Q;
  a.h = e.h_v;
  a.NB = NB;
  a.msg_sum = e.msg_sum;
  a.log_probs = log_probs;
  a.L = L;
  a.K = K;
  HK_CHECK(launch_teacher_forced(ctx->model, a, s), "teacher-forced launch failed");
  return HKBS_OK;
}

size_t tf_bytes(int L, int K) {
  return encode_bytes(L, K) + aligned_bytes<float>((size_t)(kLayers + 1) * L * kH) + aligned_bytes<float>((size_t)L * 256);
}

// inverse_fold_scalar.cpp:471-493 (double accumulation, residue order).
float average_nll_host(const int32_t* tokens, const float* lp, const float* chain_mask, const float* mask, int L) {
  double loss = 0.0, msum = 0.0;
  for (int r = 0; r < L; ++r) {
    const float active = (chain_mask ? chain_mask[r] : 1.0F) * mask[r];
    if (active == 0.0F) continue;
    const int32_t t = tokens[r];
    if (t < 0 || t >= kV) continue;
    loss -= static_cast<double>(lp[(size_t)r * kV + t]);
    msum += static_cast<double>(active);
  }
  return msum > 0.0 ? static_cast<float>(loss / msum) : 0.0F;
}

bool tokens_valid(const int32_t* tokens, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (tokens[i] < 0 || tokens[i] >= kV) return false;
  return true;
}

}  // namespace

extern "C" {

hkbs_status hkbs_pmpnn_score(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                             const int32_t* residue_indices, const int32_t* chain_labels, const float* chain_mask,
                             const int32_t* tokens, const int32_t* order, int32_t L, float* log_probs, float* score) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (L < 0) return fail(HKBS_INVALID_ARGUMENT, "residue count is negative");
  if (L > 0 && (!coords || !atom_sources)) return fail(HKBS_INVALID_ARGUMENT, "ProteinMPNN inverse fold coordinates pointer is null");
  if (!log_probs) return fail(HKBS_INVALID_ARGUMENT, "ProteinMPNN teacher-forced output shape is invalid");
  if (L > 0 && !tokens) return fail(HKBS_INVALID_ARGUMENT, "ProteinMPNN token pointer is null");
  if (!tokens_valid(tokens, (size_t)L)) return fail(HKBS_INVALID_ARGUMENT, "ProteinMPNN token id is outside the v48 vocabulary");
  if (L == 0) {
    if (score) *score = 0.0F;
    return HKBS_OK;
  }
  std::vector<int32_t> pos(L);
  if (order) {
    if (!is_permutation(order, L)) return fail(HKBS_INVALID_ARGUMENT, "ProteinMPNN input decoding_order must be a permutation");
    for (int p = 0; p < L; ++p) pos[order[p]] = p;
  } else {
    std::iota(pos.begin(), pos.end(), 0);
  }
  const int K = std::min(kKmax, L);
  DeviceArena& ar = ctx->arena;
  if (ar.reserve(input_bytes(L) + tf_bytes(L, K) + 2 * aligned_bytes<int32_t>(L) + aligned_bytes<float>((size_t)L * kV) +
                 (64u << 10), busy_event(ctx)) != hipSuccess)
    return fail(HKBS_INTERNAL_ERROR, "device workspace allocation failed");
  if ((st = after_previous_call(ctx, ctx->stream)) != HKBS_OK) return st;
  ar.reset();
  Inputs in{};
  if ((st = upload_inputs(ctx, ar, coords, atom_sources, residue_indices, chain_labels, nullptr, nullptr, L, in)) != HKBS_OK)
    return st;
  int32_t* d_tok = ar.take<int32_t>(L);
  int32_t* d_pos = ar.take<int32_t>(L);
  float* d_lp = ar.take<float>((size_t)L * kV);
  hipStream_t s = ctx->stream;
  HK_CHECK(hipMemcpyAsync(d_tok, tokens, (size_t)L * 4, hipMemcpyHostToDevice, s), "H2D failed");
  HK_CHECK(hipMemcpyAsync(d_pos, pos.data(), (size_t)L * 4, hipMemcpyHostToDevice, s), "H2D failed");
  if ((st = teacher_forced_chunk(ctx, in.coords, in.src, in.resid, in.chain, d_tok, d_pos, L, K, nullptr, nullptr, d_lp,
                                 ar)) != HKBS_OK)
    return st;
  HK_CHECK(hipMemcpyAsync(log_probs, d_lp, (size_t)L * kV * 4, hipMemcpyDeviceToHost, s), "D2H failed");
  HK_CHECK(hipStreamSynchronize(s), "teacher-forced kernels failed");
  if (score) {
    std::vector<float> mask;
    residue_mask_host(atom_sources, L, mask);
    *score = average_nll_host(tokens, log_probs, chain_mask, mask.data(), L);
  }
  return HKBS_OK;
}

hkbs_status hkbs_pmpnn_score_batch(hkbs_pmpnn* ctx, int32_t n, const int64_t* offsets, const float* coords,
                                   const uint8_t* atom_sources, const int32_t* tokens, const int32_t* orders,
                                   float* log_probs, float* scores) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (n < 0 || !offsets) return fail(HKBS_INVALID_ARGUMENT, "ragged batch offsets are missing");
  if (n == 0) return HKBS_OK;
  if (offsets[0] != 0) return fail(HKBS_INVALID_ARGUMENT, "ragged batch offsets must start at 0");
  for (int i = 0; i < n; ++i)
    if (offsets[i + 1] <= offsets[i]) return fail(HKBS_INVALID_ARGUMENT, "ragged batch proteins must be non-empty");
  const int64_t total = offsets[n];
  if (total > (int64_t)1 << 30) return fail(HKBS_INVALID_ARGUMENT, "ragged batch is too large");
  if (!coords || !atom_sources || !tokens || !log_probs)
    return fail(HKBS_INVALID_ARGUMENT, "ragged batch pointers must be non-null");
  if (!tokens_valid(tokens, (size_t)total)) return fail(HKBS_INVALID_ARGUMENT, "ProteinMPNN token id is outside the v48 vocabulary");
  std::vector<int32_t> pos((size_t)total);
  for (int i = 0; i < n; ++i) {
    const int64_t o = offsets[i];
    const int L = static_cast<int>(offsets[i + 1] - o);
    if (orders) {
      if (!is_permutation(orders + o, L)) return fail(HKBS_INVALID_ARGUMENT, "ProteinMPNN input decoding_order must be a permutation");
      for (int p = 0; p < L; ++p) pos[(size_t)o + orders[o + p]] = p;
    } else {
      for (int p = 0; p < L; ++p) pos[(size_t)o + p] = p;
    }
  }
  // Chunks of consecutive proteins with the same K = min(48, L), bounded in edges
  // (HKBS_SCORE_CHUNK_EDGES lowers the bound, so that tests can reach several chunks).
  size_t kChunkEdges = (size_t)4 << 20;
  if (const char* env = std::getenv("HKBS_SCORE_CHUNK_EDGES"))
    kChunkEdges = std::max<size_t>(1, std::min<size_t>(kChunkEdges, std::strtoull(env, nullptr, 10)));
  struct Chunk { int first, last; int64_t r0, r1; int K; };
  std::vector<Chunk> chunks;
  for (int i = 0; i < n;) {
    const int K = (int)std::min<int64_t>(kKmax, offsets[i + 1] - offsets[i]);
    int j = i + 1;
    while (j < n && std::min<int64_t>(kKmax, offsets[j + 1] - offsets[j]) == K &&
           (size_t)(offsets[j + 1] - offsets[i]) * K <= kChunkEdges)
      ++j;
    chunks.push_back({i, j, offsets[i], offsets[j], K});
    i = j;
  }
  // Two staging slots: chunk c uses slot c % 2 (pinned host buffers and device input / log-prob buffers),
  // so that chunk c + 1's inputs go up while chunk c computes and chunk c's log-probs come down while
  // chunk c + 1 computes. The encoder and decoder workspace after the slots is shared (one compute stream).
  int maxL = 0, maxP = 0;
  size_t work = 0;
  for (const Chunk& ch : chunks) {
    const int L = (int)(ch.r1 - ch.r0);
    maxL = std::max(maxL, L);
    maxP = std::max(maxP, ch.last - ch.first);
    work = std::max(work, tf_bytes(L, ch.K));
  }
  const size_t Lm = (size_t)maxL;
  const size_t slot_dev = aligned_bytes<float>(Lm * 15) + aligned_bytes<uint8_t>(Lm * 5) + 3 * aligned_bytes<int32_t>(Lm) +
                          aligned_bytes<int64_t>((size_t)maxP + 1) + aligned_bytes<float>(Lm * kV);
  // Nothing of an earlier call (one that returned early included) may still
  // use the staging slots or the workspace.
  hipStream_t s = ctx->stream;
  for (hipStream_t st2 : {s, ctx->side, ctx->down})
    if (st2) HK_CHECK(hipStreamSynchronize(st2), "an earlier call's kernels failed");
  if (ctx->done_recorded) HK_CHECK(hipEventSynchronize(ctx->done), "an earlier call's kernels failed");
  DeviceArena& ar = ctx->arena;
  if (ar.reserve(2 * slot_dev + work + (64u << 10), nullptr) != hipSuccess)
    return fail(HKBS_INTERNAL_ERROR, "device workspace allocation failed");
  struct Slot {
    float* coords;
    uint8_t* src;
    int32_t *tok, *pos, *seg;
    int64_t* off;
    float* lp;
  };
  auto take_slot = [&](auto&& take) {
    Slot sl{};
    sl.coords = take(sl.coords, Lm * 15);
    sl.src = take(sl.src, Lm * 5);
    sl.tok = take(sl.tok, Lm);
    sl.pos = take(sl.pos, Lm);
    sl.seg = take(sl.seg, Lm);
    sl.off = take(sl.off, (size_t)maxP + 1);
    sl.lp = take(sl.lp, Lm * kV);
    return sl;
  };
  ar.reset();
  Slot dev[2];
  for (Slot& sl : dev) sl = take_slot([&](auto* p, size_t n) { return ar.take<std::remove_pointer_t<decltype(p)>>(n); });
  const size_t mark = ar.used;
  if (ctx->pinned_cap < 2 * slot_dev) {
    if (ctx->pinned) (void)hipHostFree(ctx->pinned);
    ctx->pinned = nullptr;
    ctx->pinned_cap = 0;
    if (hipHostMalloc(reinterpret_cast<void**>(&ctx->pinned), 2 * slot_dev, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      ctx->pinned = nullptr;
      return fail(HKBS_INTERNAL_ERROR, "pinned staging allocation failed");
    }
    ctx->pinned_cap = 2 * slot_dev;
  }
  if (!ctx->down && hipStreamCreateWithFlags(&ctx->down, hipStreamNonBlocking) != hipSuccess) {
    ctx->down = nullptr;
    return fail(HKBS_INTERNAL_ERROR, "HIP stream creation failed");
  }
  for (auto& evs : ctx->score_ev)
    for (hipEvent_t& ev : evs)
      if (!ev && hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
        ev = nullptr;
        return fail(HKBS_INTERNAL_ERROR, "HIP event creation failed");
      }
  Slot pin[2];
  {
    size_t at = 0;
    for (Slot& sl : pin)
      sl = take_slot([&](auto* p, size_t n) {
        auto* q = reinterpret_cast<decltype(p)>(ctx->pinned + at);
        at += aligned_bytes<std::remove_pointer_t<decltype(p)>>(n);
        return q;
      });
  }
  hipEvent_t* uploaded = ctx->score_ev[0];
  hipEvent_t* computed = ctx->score_ev[1];
  hipEvent_t* copied = ctx->score_ev[2];
  // chunk c's log-probs from its slot's pinned buffer to the caller's (its copy has been waited for)
  auto deliver = [&](int c) {
    const Chunk& ch = chunks[c];
    std::memcpy(log_probs + ch.r0 * kV, pin[c & 1].lp, (size_t)(ch.r1 - ch.r0) * kV * sizeof(float));
  };
  const int nch = static_cast<int>(chunks.size());
  for (int c = 0; c < nch; ++c) {
    const Chunk& ch = chunks[c];
    const int L = (int)(ch.r1 - ch.r0);
    const int np = ch.last - ch.first;
    const int k = c & 1;
    Slot& hp = pin[k];
    Slot& dp = dev[k];
    if (c >= 2) {
      // chunk c - 2 (same slot): its results are down, so its pinned and device buffers are free
      HK_CHECK(hipEventSynchronize(copied[k]), "teacher-forced kernels failed");
      deliver(c - 2);
    }
    std::memcpy(hp.coords, coords + ch.r0 * 15, (size_t)L * 15 * sizeof(float));
    std::memcpy(hp.src, atom_sources + ch.r0 * 5, (size_t)L * 5);
    std::memcpy(hp.tok, tokens + ch.r0, (size_t)L * 4);
    std::memcpy(hp.pos, pos.data() + ch.r0, (size_t)L * 4);
    for (int p = 0; p < np; ++p) {
      hp.off[p] = offsets[ch.first + p] - ch.r0;
      for (int64_t r = offsets[ch.first + p]; r < offsets[ch.first + p + 1]; ++r) hp.seg[r - ch.r0] = p;
    }
    hp.off[np] = L;
    hipStream_t up = ctx->side;
    HK_CHECK(hipMemcpyAsync(dp.coords, hp.coords, (size_t)L * 15 * sizeof(float), hipMemcpyHostToDevice, up), "H2D failed");
    HK_CHECK(hipMemcpyAsync(dp.src, hp.src, (size_t)L * 5, hipMemcpyHostToDevice, up), "H2D failed");
    HK_CHECK(hipMemcpyAsync(dp.tok, hp.tok, (size_t)L * 4, hipMemcpyHostToDevice, up), "H2D failed");
    HK_CHECK(hipMemcpyAsync(dp.pos, hp.pos, (size_t)L * 4, hipMemcpyHostToDevice, up), "H2D failed");
    HK_CHECK(hipMemcpyAsync(dp.seg, hp.seg, (size_t)L * 4, hipMemcpyHostToDevice, up), "H2D failed");
    HK_CHECK(hipMemcpyAsync(dp.off, hp.off, (size_t)(np + 1) * 8, hipMemcpyHostToDevice, up), "H2D failed");
    HK_CHECK(hipEventRecord(uploaded[k], up), "event record failed");
    HK_CHECK(hipStreamWaitEvent(s, uploaded[k], 0), "stream wait failed");
    ar.used = mark;
    if ((st = teacher_forced_chunk(ctx, dp.coords, dp.src, nullptr, nullptr, dp.tok, dp.pos, L, ch.K, dp.seg, dp.off,
                                   dp.lp, ar)) != HKBS_OK)
      return st;
    HK_CHECK(hipEventRecord(computed[k], s), "event record failed");
    HK_CHECK(hipStreamWaitEvent(ctx->down, computed[k], 0), "stream wait failed");
    HK_CHECK(hipMemcpyAsync(hp.lp, dp.lp, (size_t)L * kV * sizeof(float), hipMemcpyDeviceToHost, ctx->down), "D2H failed");
    HK_CHECK(hipEventRecord(copied[k], ctx->down), "event record failed");
    // The next upload into this slot's device inputs (chunk c + 2) comes after this chunk's results are down,
    // which follow its kernels, so the kernels have read the inputs by then.
  }
  for (int c = std::max(0, nch - 2); c < nch; ++c) {
    HK_CHECK(hipEventSynchronize(copied[c & 1]), "teacher-forced kernels failed");
    deliver(c);
  }
  HK_CHECK(hipStreamSynchronize(s), "teacher-forced kernels failed");
  if (scores) {
    std::vector<float> mask;
    for (int i = 0; i < n; ++i) {
      const int64_t o = offsets[i];
      const int L = static_cast<int>(offsets[i + 1] - o);
      residue_mask_host(atom_sources + o * 5, L, mask);
      scores[i] = average_nll_host(tokens + o, log_probs + o * kV, nullptr, mask.data(), L);
    }
  }
  return HKBS_OK;
}

hkbs_status hkbs_pmpnn_knn(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources, int32_t L, int32_t* idx,
                           float* d2) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (L < 0) return fail(HKBS_INVALID_ARGUMENT, "residue count is negative");
  if (L == 0) return HKBS_OK;
  if (!coords || !atom_sources || !idx || !d2) return fail(HKBS_INVALID_ARGUMENT, "kNN pointers must be non-null");
  const int K = std::min(kKmax, L);
  const size_t S = (size_t)L * K;
  DeviceArena& ar = ctx->arena;
  if (ar.reserve(input_bytes(L) + encode_bytes(L, K) + (64u << 10), busy_event(ctx)) != hipSuccess)
    return fail(HKBS_INTERNAL_ERROR, "device workspace allocation failed");
  if ((st = after_previous_call(ctx, ctx->stream)) != HKBS_OK) return st;
  ar.reset();
  Inputs in{};
  if ((st = upload_inputs(ctx, ar, coords, atom_sources, nullptr, nullptr, nullptr, nullptr, L, in)) != HKBS_OK) return st;
  EncodeBuffers e = take_encode(ar, L, K);
  HK_CHECK(launch_knn(in.coords, in.src, L, K, e.idx, e.d2, e.mask, e.ca, ctx->stream), "kNN launch failed");
  HK_CHECK(hipMemcpyAsync(idx, e.idx, S * 4, hipMemcpyDeviceToHost, ctx->stream), "D2H failed");
  HK_CHECK(hipMemcpyAsync(d2, e.d2, S * 4, hipMemcpyDeviceToHost, ctx->stream), "D2H failed");
  HK_CHECK(hipStreamSynchronize(ctx->stream), "kNN kernel failed");
  return HKBS_OK;
}

hkbs_status hkbs_pmpnn_encode(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                              const int32_t* residue_indices, const int32_t* chain_labels, int32_t L, float* mask,
                              int32_t* idx, float* h_v, float* h_e) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (L < 0) return fail(HKBS_INVALID_ARGUMENT, "residue count is negative");
  if (L == 0) return HKBS_OK;
  if (!coords || !atom_sources) return fail(HKBS_INVALID_ARGUMENT, "encoder structure pointers must be non-null");
  const int K = std::min(kKmax, L);
  const size_t S = (size_t)L * K;
  DeviceArena& ar = ctx->arena;
  if (ar.reserve(input_bytes(L) + encode_bytes(L, K) + (64u << 10), busy_event(ctx)) != hipSuccess)
    return fail(HKBS_INTERNAL_ERROR, "device workspace allocation failed");
  if ((st = after_previous_call(ctx, ctx->stream)) != HKBS_OK) return st;
  ar.reset();
  Inputs in{};
  if ((st = upload_inputs(ctx, ar, coords, atom_sources, residue_indices, chain_labels, nullptr, nullptr, L, in)) != HKBS_OK)
    return st;
  EncodeBuffers e = take_encode(ar, L, K);
  HK_CHECK(run_encode(ctx, in.coords, in.src, in.resid, in.chain, L, K, e), "encoder launch failed");
  hipStream_t s = ctx->stream;
  if (mask) HK_CHECK(hipMemcpyAsync(mask, e.mask, (size_t)L * 4, hipMemcpyDeviceToHost, s), "D2H failed");
  if (idx) HK_CHECK(hipMemcpyAsync(idx, e.idx, S * 4, hipMemcpyDeviceToHost, s), "D2H failed");
  if (h_v) HK_CHECK(hipMemcpyAsync(h_v, e.h_v, (size_t)L * kH * 4, hipMemcpyDeviceToHost, s), "D2H failed");
  if (h_e) HK_CHECK(hipMemcpyAsync(h_e, e.h_e, S * kH * 4, hipMemcpyDeviceToHost, s), "D2H failed");
  HK_CHECK(hipStreamSynchronize(s), "encoder kernels failed");
  return HKBS_OK;
}

hkbs_status hkbs_pmpnn_edge_features(hkbs_pmpnn* ctx, const float* coords, const uint8_t* atom_sources,
                                     const int32_t* residue_indices, const int32_t* chain_labels, int32_t L,
                                     float* features) {
  hkbs_status st = enter(ctx);
  if (st != HKBS_OK) return st;
  if (L < 0) return fail(HKBS_INVALID_ARGUMENT, "residue count is negative");
  if (L == 0) return HKBS_OK;
  if (!coords || !atom_sources || !features) return fail(HKBS_INVALID_ARGUMENT, "feature pointers must be non-null");
  const int K = std::min(kKmax, L);
  const size_t S = (size_t)L * K;
  DeviceArena& ar = ctx->arena;
  if (ar.reserve(input_bytes(L) + encode_bytes(L, K) + aligned_bytes<float>(S * kEdgeIn) + (64u << 10), busy_event(ctx)) != hipSuccess)
    return fail(HKBS_INTERNAL_ERROR, "device workspace allocation failed");
  if ((st = after_previous_call(ctx, ctx->stream)) != HKBS_OK) return st;
  ar.reset();
  Inputs in{};
  if ((st = upload_inputs(ctx, ar, coords, atom_sources, residue_indices, chain_labels, nullptr, nullptr, L, in)) != HKBS_OK)
    return st;
  EncodeBuffers e = take_encode(ar, L, K);
  float* f = ar.take<float>(S * kEdgeIn);
  HK_CHECK(launch_knn(in.coords, in.src, L, K, e.idx, e.d2, e.mask, e.ca, ctx->stream), "kNN launch failed");
  HK_CHECK(launch_edge_features(ctx->model, in.coords, in.src, in.resid, in.chain, e.idx, L, K, f, ctx->stream),
           "feature launch failed");
  HK_CHECK(hipMemcpyAsync(features, f, S * kEdgeIn * 4, hipMemcpyDeviceToHost, ctx->stream), "D2H failed");
  HK_CHECK(hipStreamSynchronize(ctx->stream), "feature kernels failed");
  return HKBS_OK;
}

}  // extern "C"
