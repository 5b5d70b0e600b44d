// The LM head's tensors from the reference's weight store (src/core/weights.cpp:
// 13-58): a consolidated <root>.safetensors when that file exists, else one
// <root>/<name>.npy per tensor. The head reads final_norm.weight,
// final_norm.bias, semantic_head.weight ([V][D], the Linear's (out, in)) and
// semantic_head.bias (src/t2s/text2semantic.cpp:114-115).
//
// Host code: the files are parsed here (npy versions 1-3 with little-endian
// f2/f4/f8 or u4 data, C order; safetensors with F16/BF16/F32/F64/U32 data),
// converted to the storage the caller asks for and copied to the device once.
// 8-bit storage either comes from the file (an 8-bit quantized head: u32
// weight words holding four codes each, least significant byte first, with
// semantic_head.scales and semantic_head.biases of [V][D / group]) or is made
// here: per group of `group` inputs, bias = min, scale = (max - min) / 255
// (1 when max == min), q = round((w - bias) / scale) clamped to 0..255.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <new>
#include <string>
#include <sys/stat.h>
#include <vector>

#include "../../include/c4s_sampling.h"

namespace {

// Largest dimension, and largest element count, a tensor of the store may have
// (far above an LM head's; the checks keep products and offsets from overflowing).
constexpr int64_t kMaxDim = (int64_t)1 << 31;
constexpr int64_t kMaxCount = (int64_t)1 << 36;

struct Tensor {
  std::vector<float> f;        // values as fp32 (float data)
  std::vector<uint32_t> u;     // u32 data (packed 8-bit codes)
  std::vector<int64_t> shape;
  bool is_u32 = false;
  int64_t count() const {      // valid once shape_ok() held
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
  // every dimension in [1, kMaxDim] and at most kMaxCount elements
  bool shape_ok() const {
    int64_t n = 1;
    for (int64_t d : shape) {
      if (d < 1 || d > kMaxDim) return false;
      n *= d;
      if (n > kMaxCount) return false;
    }
    return true;
  }
};

// Decimal digits as a non-negative integer; false past `limit` (no overflow).
bool parse_count(const std::string& digits, int64_t limit, int64_t& out) {
  out = 0;
  if (digits.empty()) return false;
  for (char ch : digits) {
    if (ch < '0' || ch > '9') return false;
    if (out > (limit - (ch - '0')) / 10) return false;
    out = 10 * out + (ch - '0');
  }
  return true;
}

// Every decimal number of `list` in order (a shape tuple or a JSON list);
// false when one exceeds `limit`.
bool parse_ints(const std::string& list, int64_t limit, std::vector<int64_t>& v) {
  v.clear();
  std::string num;
  for (size_t i = 0; i <= list.size(); ++i) {
    const char ch = i < list.size() ? list[i] : ' ';
    if (ch >= '0' && ch <= '9') {
      num += ch;
    } else if (!num.empty()) {
      int64_t x;
      if (!parse_count(num, limit, x)) return false;
      v.push_back(x);
      num.clear();
    }
  }
  return true;
}

bool read_file(const std::string& path, std::vector<char>& buf) {
  std::FILE* fp = std::fopen(path.c_str(), "rb");
  if (!fp) return false;
  std::fseek(fp, 0, SEEK_END);
  const long n = std::ftell(fp);
  std::fseek(fp, 0, SEEK_SET);
  buf.resize(n > 0 ? (size_t)n : 0);
  const size_t got = n > 0 ? std::fread(buf.data(), 1, buf.size(), fp) : 0;
  std::fclose(fp);
  return got == buf.size();
}

bool is_file(const std::string& p) {
  struct stat st {};
  return stat(p.c_str(), &st) == 0 && (st.st_mode & S_IFREG);
}

// IEEE binary16 to binary32 (every half value is exact in fp32).
float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const int exp = (h >> 10) & 0x1F;
  const uint32_t man = h & 0x3FF;
  float v;
  if (exp == 0) v = std::ldexp((float)man, -24);                 // zero and subnormals
  else if (exp == 31) v = man ? NAN : INFINITY;
  else v = std::ldexp((float)(man | 0x400), exp - 25);
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  bits |= sign;
  std::memcpy(&v, &bits, 4);
  return v;
}

float bf16_to_float(uint16_t b) {
  const uint32_t bits = (uint32_t)b << 16;
  float v;
  std::memcpy(&v, &bits, 4);
  return v;
}

// Element kinds both formats name.
enum Kind { kF16, kBF16, kF32, kF64, kU32, kBad };

bool convert(const char* data, size_t bytes, Kind kind, Tensor& t, std::string& err) {
  if (!t.shape_ok()) {
    err = "a dimension is zero or too large";
    return false;
  }
  const int64_t n = t.count();
  const size_t es = kind == kF64 ? 8 : (kind == kF32 || kind == kU32) ? 4 : 2;
  if ((size_t)n * es != bytes) {
    err = "data size does not match the shape";
    return false;
  }
  if (kind == kU32) {
    t.is_u32 = true;
    t.u.resize(n);
    std::memcpy(t.u.data(), data, bytes);
    return true;
  }
  t.f.resize(n);
  for (int64_t i = 0; i < n; ++i) {
    const char* p = data + i * es;
    if (kind == kF32) {
      std::memcpy(&t.f[i], p, 4);
    } else if (kind == kF64) {
      double d;
      std::memcpy(&d, p, 8);
      t.f[i] = (float)d;
    } else {
      uint16_t h;
      std::memcpy(&h, p, 2);
      t.f[i] = kind == kF16 ? half_to_float(h) : bf16_to_float(h);
    }
  }
  return true;
}

// ---- .npy (numpy.lib.format: magic, version, header length, a Python dict) -------

std::string dict_field(const std::string& h, const std::string& key) {
  const size_t k = h.find("'" + key + "'");
  if (k == std::string::npos) return "";
  size_t p = h.find(':', k);
  if (p == std::string::npos) return "";
  ++p;
  while (p < h.size() && h[p] == ' ') ++p;
  if (p < h.size() && h[p] == '(') return h.substr(p, h.find(')', p) - p + 1);
  return h.substr(p, h.find_first_of(",}", p) - p);
}

bool parse_npy(const std::vector<char>& f, Tensor& t, std::string& err) {
  if (f.size() < 10 || std::memcmp(f.data(), "\x93NUMPY", 6) != 0) {
    err = "not a .npy file";
    return false;
  }
  const int major = (unsigned char)f[6];
  size_t hlen, pre;
  if (major == 1) {
    hlen = (unsigned char)f[8] | ((size_t)(unsigned char)f[9] << 8);
    pre = 10;
  } else {
    if (f.size() < 12) { err = "truncated .npy header"; return false; }
    hlen = 0;
    for (int i = 0; i < 4; ++i) hlen |= (size_t)(unsigned char)f[8 + i] << (8 * i);
    pre = 12;
  }
  if (pre + hlen > f.size()) { err = "truncated .npy header"; return false; }
  const std::string h(f.data() + pre, hlen);
  const std::string descr = dict_field(h, "descr");
  if (dict_field(h, "fortran_order").find("False") == std::string::npos) {
    err = "fortran_order .npy is not supported";
    return false;
  }
  Kind kind = kBad;
  if (descr.find("<f4") != std::string::npos) kind = kF32;
  else if (descr.find("<f8") != std::string::npos) kind = kF64;
  else if (descr.find("<f2") != std::string::npos) kind = kF16;
  else if (descr.find("<u4") != std::string::npos) kind = kU32;
  if (kind == kBad) { err = "unsupported .npy dtype " + descr; return false; }
  if (!parse_ints(dict_field(h, "shape"), kMaxDim, t.shape)) { err = "bad .npy shape"; return false; }
  const size_t off = pre + hlen;
  return convert(f.data() + off, f.size() - off, kind, t, err);
}

// ---- .safetensors (u64 header length, a JSON header, the data) -------------------

// The JSON value of `key` inside the object text `obj`: a string or a [...] list.
std::string json_field(const std::string& obj, const std::string& key) {
  const size_t k = obj.find("\"" + key + "\"");
  if (k == std::string::npos) return "";
  size_t p = obj.find(':', k);
  if (p == std::string::npos) return "";
  ++p;
  while (p < obj.size() && (obj[p] == ' ' || obj[p] == '\n' || obj[p] == '\t' || obj[p] == '\r')) ++p;
  if (p >= obj.size()) return "";
  if (obj[p] == '"') return obj.substr(p + 1, obj.find('"', p + 1) - p - 1);
  if (obj[p] == '[') return obj.substr(p, obj.find(']', p) - p + 1);
  return "";
}

bool parse_safetensors(const std::vector<char>& f, const std::string& name, Tensor& t, std::string& err) {
  if (f.size() < 8) { err = "not a .safetensors file"; return false; }
  uint64_t n = 0;
  for (int i = 0; i < 8; ++i) n |= (uint64_t)(unsigned char)f[i] << (8 * i);
  if (n > f.size() - 8) { err = "truncated .safetensors header"; return false; }
  const std::string h(f.data() + 8, n);
  // the tensor's key: the quoted name followed (after blanks) by a colon
  size_t k = 0;
  for (;;) {
    k = h.find("\"" + name + "\"", k);
    if (k == std::string::npos) { err = "no tensor " + name; return false; }
    size_t p = k + name.size() + 2;
    while (p < h.size() && (h[p] == ' ' || h[p] == '\n' || h[p] == '\t' || h[p] == '\r')) ++p;
    if (p < h.size() && h[p] == ':') { k = p; break; }
    k += 1;
  }
  const size_t o0 = h.find('{', k), o1 = h.find('}', o0);
  if (o0 == std::string::npos || o1 == std::string::npos) { err = "bad .safetensors header"; return false; }
  const std::string obj = h.substr(o0, o1 - o0 + 1);
  const std::string dt = json_field(obj, "dtype");
  Kind kind = dt == "F32" ? kF32 : dt == "F16" ? kF16 : dt == "BF16" ? kBF16 : dt == "F64" ? kF64 :
              dt == "U32" ? kU32 : kBad;
  if (kind == kBad) { err = "unsupported .safetensors dtype " + dt; return false; }
  std::vector<int64_t> off;
  if (!parse_ints(json_field(obj, "shape"), kMaxDim, t.shape) ||
      !parse_ints(json_field(obj, "data_offsets"), (int64_t)f.size(), off) || off.size() != 2 || off[1] < off[0] ||
      (uint64_t)off[1] > f.size() - 8 - n) {
    err = "bad data_offsets for " + name;
    return false;
  }
  return convert(f.data() + 8 + n + off[0], (size_t)(off[1] - off[0]), kind, t, err);
}

// One tensor of the store rooted at `root` (weights.cpp:13-58).
bool load_tensor(const std::string& root_in, const std::string& name, Tensor& t, std::string& err) {
  std::string root = root_in;
  if (!root.empty() && root.back() == '/') root.pop_back();
  std::vector<char> buf;
  const std::string st = root + ".safetensors";
  if (is_file(st)) {
    if (!read_file(st, buf)) { err = "cannot read " + st; return false; }
    if (!parse_safetensors(buf, name, t, err)) { err = st + ": " + err; return false; }
    return true;
  }
  const std::string np = root + "/" + name + ".npy";
  if (!read_file(np, buf)) { err = "no " + st + " and cannot read " + np; return false; }
  if (!parse_npy(buf, t, err)) { err = np + ": " + err; return false; }
  return true;
}

uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

thread_local std::string g_err;

int fail(const std::string& e) {
  g_err = e;
  return C4S_EINVAL;
}

template <class T>
int upload(const std::vector<T>& h, void** d) {
  *d = nullptr;
  if (hipMalloc(d, h.size() * sizeof(T)) != hipSuccess) return C4S_EHIP;
  if (hipMemcpy(*d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) return C4S_EHIP;
  return C4S_OK;
}

}  // namespace

extern "C" {

const char* c4s_weights_last_error(void) { return g_err.c_str(); }

namespace {
int tensor_read_f32(const char* root, const char* name, float* out, int64_t cap, int64_t* shape, int32_t* ndim) {
  if (!root || !name || !ndim) return fail("tensor_read: NULL argument");
  Tensor t;
  std::string err;
  if (!load_tensor(root, name, t, err)) return fail(err);
  if (t.is_u32) return fail(std::string("tensor_read: ") + name + " holds integer codes");
  if ((int)t.shape.size() > 8) return fail("tensor_read: more than 8 dimensions");
  *ndim = (int32_t)t.shape.size();
  if (shape)
    for (size_t i = 0; i < t.shape.size(); ++i) shape[i] = t.shape[i];
  if (out) {
    if (cap < t.count()) return fail("tensor_read: output capacity below the tensor's size");
    std::memcpy(out, t.f.data(), t.f.size() * sizeof(float));
  }
  return C4S_OK;
}

int head_weights_load(const char* root, int32_t wdtype, int32_t group, c4s_head_weights* out) {
  if (!root || !out) return fail("head_weights_load: NULL argument");
  std::memset(out, 0, sizeof(*out));
  if (wdtype != C4S_W_BF16 && wdtype != C4S_W_F32 && wdtype != C4S_W_Q8)
    return fail("head_weights_load: unknown weight dtype");
  Tensor g, b, w, bias;
  std::string err;
  if (!load_tensor(root, "final_norm.weight", g, err) || !load_tensor(root, "final_norm.bias", b, err) ||
      !load_tensor(root, "semantic_head.weight", w, err) || !load_tensor(root, "semantic_head.bias", bias, err))
    return fail(err);
  if (g.shape.size() != 1 || b.shape != g.shape || bias.shape.size() != 1 || w.shape.size() != 2)
    return fail("head_weights_load: expected final_norm.* of [D], semantic_head.weight of [V][D or D/4], "
                "semantic_head.bias of [V]");
  const int64_t D = g.shape[0], V = bias.shape[0];
  if (g.is_u32 || b.is_u32 || bias.is_u32) return fail("head_weights_load: integer LayerNorm or bias tensor");
  if (D < 32 || D % 32 != 0 || D > (1 << 24) || V < 1 || V > (1 << 24))
    return fail("head_weights_load: D must be a positive multiple of 32");
  std::vector<uint8_t> q;
  std::vector<float> qs, qb;
  if (w.is_u32) {   // an 8-bit quantized head: four codes a word
    if (wdtype != C4S_W_Q8) return fail("head_weights_load: the file holds 8-bit codes; ask for C4S_W_Q8");
    if (w.shape[0] != V || w.shape[1] * 4 != D) return fail("head_weights_load: packed weight is not [V][D/4]");
    Tensor s, o;
    if (!load_tensor(root, "semantic_head.scales", s, err) || !load_tensor(root, "semantic_head.biases", o, err))
      return fail(err);
    if (s.shape.size() != 2 || s.shape[0] != V || o.shape != s.shape || s.shape[1] < 1 || D % s.shape[1] != 0)
      return fail("head_weights_load: scales / biases are not [V][D/group]");
    group = (int32_t)(D / s.shape[1]);
    q.resize((size_t)V * D);
    for (size_t i = 0; i < w.u.size(); ++i)
      for (int j = 0; j < 4; ++j) q[4 * i + j] = (uint8_t)(w.u[i] >> (8 * j));
    qs = s.f;
    qb = o.f;
  } else {
    if (w.shape[0] != V || w.shape[1] != D) return fail("head_weights_load: semantic_head.weight is not [V][D]");
    if (wdtype == C4S_W_Q8) {
      if ((group != 32 && group != 64 && group != 128) || D % group != 0)
        return fail("head_weights_load: group must be 32, 64 or 128 and divide D");
      const int64_t ng = D / group;
      q.resize((size_t)V * D);
      qs.resize((size_t)V * ng);
      qb.resize((size_t)V * ng);
      for (int64_t n = 0; n < V; ++n)
        for (int64_t k = 0; k < ng; ++k) {
          const float* p = &w.f[(size_t)n * D + k * group];
          double lo = p[0], hi = p[0];
          for (int i = 1; i < group; ++i) { lo = std::fmin(lo, p[i]); hi = std::fmax(hi, p[i]); }
          const double sc = hi > lo ? (hi - lo) / 255.0 : 1.0;
          for (int i = 0; i < group; ++i)
            q[(size_t)n * D + k * group + i] = (uint8_t)std::fmin(255.0, std::fmax(0.0, std::nearbyint((p[i] - lo) / sc)));
          qs[(size_t)n * ng + k] = (float)sc;
          qb[(size_t)n * ng + k] = (float)lo;
        }
    }
  }
  if (wdtype == C4S_W_Q8 && (group != 32 && group != 64 && group != 128))
    return fail("head_weights_load: the file's group size is not 32, 64 or 128");
  out->D = (int32_t)D;
  out->V = (int32_t)V;
  out->wdtype = wdtype;
  out->group = wdtype == C4S_W_Q8 ? group : 0;
  int rc = upload(g.f, reinterpret_cast<void**>(&out->gamma));
  if (!rc) rc = upload(b.f, reinterpret_cast<void**>(&out->beta));
  if (!rc) rc = upload(bias.f, reinterpret_cast<void**>(&out->bias));
  if (!rc) {
    if (wdtype == C4S_W_F32) {
      rc = upload(w.f, &out->weight);
    } else if (wdtype == C4S_W_BF16) {
      std::vector<uint16_t> h(w.f.size());
      for (size_t i = 0; i < h.size(); ++i) h[i] = f32_to_bf16_rne(w.f[i]);
      rc = upload(h, &out->weight);
    } else {
      rc = upload(q, &out->weight);
      if (!rc) rc = upload(qs, reinterpret_cast<void**>(&out->wscale));
      if (!rc) rc = upload(qb, reinterpret_cast<void**>(&out->wbias));
    }
  }
  if (rc) {
    c4s_head_weights_free(out);
    return fail("head_weights_load: device allocation or copy failed");
  }
  return C4S_OK;
}

}  // namespace

// No exception leaves the C ABI: a malformed file that gets past the checks
// above (or an allocation that fails) is reported as C4S_EINVAL / C4S_ENOMEM.
int c4s_tensor_read_f32(const char* root, const char* name, float* out, int64_t cap, int64_t* shape,
                        int32_t* ndim) {
  try {
    return tensor_read_f32(root, name, out, cap, shape, ndim);
  } catch (const std::bad_alloc&) {
    g_err = "tensor_read: out of host memory";
    return C4S_ENOMEM;
  } catch (const std::exception& e) {
    return fail(std::string("tensor_read: ") + e.what());
  }
}

int c4s_head_weights_load(const char* root, int32_t wdtype, int32_t group, c4s_head_weights* out) {
  try {
    return head_weights_load(root, wdtype, group, out);
  } catch (const std::bad_alloc&) {
    if (out) c4s_head_weights_free(out);
    g_err = "head_weights_load: out of host memory";
    return C4S_ENOMEM;
  } catch (const std::exception& e) {
    if (out) c4s_head_weights_free(out);
    return fail(std::string("head_weights_load: ") + e.what());
  }
}

int c4s_head_weights_free(c4s_head_weights* w) {
  if (!w) return C4S_EINVAL;
  for (void* p : {(void*)w->gamma, (void*)w->beta, w->weight, (void*)w->bias, (void*)w->wscale, (void*)w->wbias})
    if (p) (void)hipFree(p);
  std::memset(w, 0, sizeof(*w));
  return C4S_OK;
}

}  // extern "C"
