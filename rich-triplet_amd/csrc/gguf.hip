// gguf.hip -- GGUF reader and weight loader (host code of librt_hip.so).
//
// Replaces GgufFile (gguf_loader.rs:156-744) and load_linear_from_gguf
// (transformer4.rs:1177-1256).  The header is parsed once through a buffered
// reader with bounds checks on every length and count; tensor bytes are read
// on demand with pread, so one handle serves several threads.  Format
// conversions run on the host, multithreaded over rows, and the result is
// uploaded to device memory in the layout the GEMV/decode kernels consume.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <exception>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/rt_gguf.h"
#include "rt_capi_util.hpp"
#include "rt_kernels.hpp"

// The reference rounds every f32 product and difference separately.
#pragma clang fp contract(off)

using rt::set_error;

namespace {

struct MetaValue {
  int32_t type = 0;
  uint64_t u = 0;      // unsigned integers and bool
  int64_t i = 0;       // signed integers
  double f = 0.0;      // f32 / f64
  std::string s;
  int32_t elem_type = -1;
  std::vector<MetaValue> arr;
};

struct TensorEntry {
  std::string name;
  int32_t n_dims = 0;
  int64_t dims[4] = {0, 0, 0, 0};
  int32_t type = -1;
  uint64_t offset = 0, n_elem = 0, n_bytes = 0;
};

// (bytes per block, elements per block): GgufType::block_info (gguf_loader.rs:106-117).
bool block_info(int32_t t, uint64_t &bpb, uint64_t &epb) {
  switch (t) {
    case RT_GGUF_F32: bpb = 4, epb = 1; return true;
    case RT_GGUF_F16: bpb = 2, epb = 1; return true;
    case RT_GGUF_BF16: bpb = 2, epb = 1; return true;
    case RT_GGUF_Q4_0: bpb = 18, epb = 32; return true;
    case RT_GGUF_Q8_0: bpb = 34, epb = 32; return true;
    case RT_GGUF_Q4_K: bpb = 144, epb = 256; return true;
    case RT_GGUF_Q5_K: bpb = 176, epb = 256; return true;
    case RT_GGUF_Q6_K: bpb = 210, epb = 256; return true;
    default: return false;
  }
}

// Buffered little-endian reader over a file descriptor.
class Reader {
 public:
  Reader(int fd, uint64_t size) : fd_(fd), size_(size), buf_(1 << 20) {}
  uint64_t pos() const { return pos_; }
  bool read(void *dst, uint64_t n) {
    uint8_t *d = static_cast<uint8_t *>(dst);
    while (n > 0) {
      if (bpos_ == blen_) {
        if (pos_ >= size_) return false;
        const ssize_t got = pread(fd_, buf_.data(), buf_.size(), (off_t)pos_);
        if (got <= 0) return false;
        bpos_ = 0, blen_ = (size_t)got;
      }
      const size_t take = (size_t)std::min<uint64_t>(n, blen_ - bpos_);
      std::memcpy(d, buf_.data() + bpos_, take);
      d += take, n -= take, bpos_ += take, pos_ += take;
    }
    return true;
  }
  template <class T>
  bool get(T &v) { return read(&v, sizeof(T)); }
  bool str(std::string &s) {
    uint64_t len;
    if (!get(len) || len > size_ - std::min(size_, pos_)) return false;
    s.resize((size_t)len);
    return read(s.data(), len);
  }
  uint64_t remaining() const { return size_ - std::min(size_, pos_); }

 private:
  int fd_;
  uint64_t size_, pos_ = 0;
  std::vector<uint8_t> buf_;
  size_t bpos_ = 0, blen_ = 0;
};

// GgufMetaValue::read_typed (gguf_loader.rs:850-878).
bool read_value(Reader &r, int32_t type, MetaValue &v, int depth) {
  v.type = type;
  switch (type) {
    case RT_GGUF_META_U8: { uint8_t x; if (!r.get(x)) return false; v.u = x; return true; }
    case RT_GGUF_META_I8: { int8_t x; if (!r.get(x)) return false; v.i = x; return true; }
    case RT_GGUF_META_U16: { uint16_t x; if (!r.get(x)) return false; v.u = x; return true; }
    case RT_GGUF_META_I16: { int16_t x; if (!r.get(x)) return false; v.i = x; return true; }
    case RT_GGUF_META_U32: { uint32_t x; if (!r.get(x)) return false; v.u = x; return true; }
    case RT_GGUF_META_I32: { int32_t x; if (!r.get(x)) return false; v.i = x; return true; }
    case RT_GGUF_META_F32: { float x; if (!r.get(x)) return false; v.f = x; return true; }
    case RT_GGUF_META_BOOL: { uint8_t x; if (!r.get(x)) return false; v.u = x != 0; return true; }
    case RT_GGUF_META_STR: return r.str(v.s);
    case RT_GGUF_META_U64: return r.get(v.u);
    case RT_GGUF_META_I64: return r.get(v.i);
    case RT_GGUF_META_F64: return r.get(v.f);
    case RT_GGUF_META_ARRAY: {
      uint32_t et;
      uint64_t n;
      if (depth > 4 || !r.get(et) || !r.get(n)) return false;
      if (n > r.remaining()) return false;  // every element takes at least one byte
      v.elem_type = (int32_t)et;
      v.arr.resize((size_t)n);
      for (auto &e : v.arr)
        if (!read_value(r, (int32_t)et, e, depth + 1)) return false;
      return true;
    }
    default: return false;
  }
}

// ---- element conversions (host) -------------------------------------------
inline float bits_to_f32(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t f32_to_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// IEEE half -> float, exact; subnormals normalised, Inf/NaN payload kept
// (f16_to_f32, gguf_loader.rs:947-976).
float half_to_float(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 0x1F) return bits_to_f32(s | 0x7F800000u | (m << 13));
  if (e != 0) return bits_to_f32(s | ((e + 112u) << 23) | (m << 13));
  if (m == 0) return bits_to_f32(s);
  // m * 2^-24 with its top bit p = 10 - lz: exponent p - 24, fraction m << lz without the top bit
  const int lz = __builtin_clz(m) - 21;
  return bits_to_f32(s | ((uint32_t)(113 - lz) << 23) | (((m << lz) & 0x3FFu) << 13));
}

// Q4KMat::f32_to_f16 (autograd2.rs:1090-1117): the low 13 mantissa bits are
// dropped (truncation toward zero), subnormal results shift without rounding.
uint16_t float_to_half_trunc(float v) {
  const uint32_t b = f32_to_bits(v), sign = (b >> 16) & 0x8000u, mant = b & 0x7FFFFFu;
  const int e = (int)((b >> 23) & 0xFFu);
  if (e == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant >> 13));
  const int he = e - 112;
  if (he >= 31) return (uint16_t)(sign | 0x7C00u);
  if (he > 0) return (uint16_t)(sign | ((uint32_t)he << 10) | (mant >> 13));
  if (he < -10) return (uint16_t)sign;
  return (uint16_t)(sign | ((mant | 0x800000u) >> (14 - he)));
}

// MatBf16::f32_to_bf16 (autograd2.rs:709-719): round to nearest even, NaN
// kept quiet.
uint16_t float_to_bf16(float v) {
  const uint32_t b = f32_to_bits(v);
  if (std::isnan(v)) return (uint16_t)((b >> 16) | 0x40u);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// Rust `x as u8`: saturating, NaN -> 0.
inline uint8_t sat_u8(float x) { return x > 0.0f ? (x >= 255.0f ? 255 : (uint8_t)x) : 0; }

// 6-bit scale/min pair j of the 12-byte packing (get_scale_min_k4).
inline void scale_min_k4(const uint8_t *sc, int j, float &s, float &m) {
  uint8_t a, b;
  if (j < 4) {
    a = sc[j] & 63;
    b = sc[j + 4] & 63;
  } else {
    a = (uint8_t)((sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4));
    b = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
  }
  s = (float)a, m = (float)b;
}

// ---- block decoders: one block into out[0 .. elems_per_block) ---------------
void dec_q4k(const uint8_t *bp, float *out) {  // gguf_loader.rs:551-621
  const float d = half_to_float(le16(bp)), dmin = half_to_float(le16(bp + 2));
  for (int c = 0; c < 4; ++c) {
    float s1, m1, s2, m2;
    scale_min_k4(bp + 4, 2 * c, s1, m1);
    scale_min_k4(bp + 4, 2 * c + 1, s2, m2);
    const float a1 = d * s1, b1 = dmin * m1, a2 = d * s2, b2 = dmin * m2;
    const uint8_t *q = bp + 16 + 32 * c;
    for (int l = 0; l < 32; ++l) {
      out[64 * c + l] = a1 * (float)(q[l] & 15) - b1;
      out[64 * c + 32 + l] = a2 * (float)(q[l] >> 4) - b2;
    }
  }
}
void dec_q5k(const uint8_t *bp, float *out) {  // gguf_loader.rs:664-743
  const float d = half_to_float(le16(bp)), dmin = half_to_float(le16(bp + 2));
  const uint8_t *qh = bp + 16, *qs = bp + 48;
  for (int c = 0; c < 4; ++c) {
    float s1, m1, s2, m2;
    scale_min_k4(bp + 4, 2 * c, s1, m1);
    scale_min_k4(bp + 4, 2 * c + 1, s2, m2);
    const float a1 = d * s1, b1 = dmin * m1, a2 = d * s2, b2 = dmin * m2;
    for (int l = 0; l < 32; ++l) {
      const uint32_t lo = (qs[32 * c + l] & 15) | (((qh[l] >> (2 * c)) & 1) << 4);
      const uint32_t hi = (qs[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4);
      out[64 * c + l] = a1 * (float)lo - b1;
      out[64 * c + 32 + l] = a2 * (float)hi - b2;
    }
  }
}
void dec_q6k(const uint8_t *bp, float *out) {  // gguf_loader.rs:482-549
  const float d = half_to_float(le16(bp + 208));
  for (int h = 0; h < 2; ++h) {
    const uint8_t *ql = bp + 64 * h, *qh = bp + 128 + 32 * h;
    const int8_t *sc = reinterpret_cast<const int8_t *>(bp + 192 + 8 * h);
    for (int l = 0; l < 32; ++l) {
      const int g = l >> 4;
      const int q[4] = {(int)((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32,
                        (int)((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32,
                        (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32,
                        (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32};
      for (int k = 0; k < 4; ++k) out[128 * h + 32 * k + l] = (d * (float)sc[g + 2 * k]) * (float)q[k];
    }
  }
}
void dec_q8_0(const uint8_t *bp, float *out) {  // gguf_loader.rs:628-650
  const float d = half_to_float(le16(bp));
  for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)bp[2 + i];
}
void dec_q4_0(const uint8_t *bp, float *out) {  // gguf_loader.rs:425-480
  const float s = half_to_float(le16(bp));
  for (int k = 0; k < 16; ++k) {
    out[k] = (float)((int)(bp[2 + k] & 15) - 8) * s;
    out[k + 16] = (float)((int)(bp[2 + k] >> 4) - 8) * s;
  }
}

// Q4KMat::quantize_block (autograd2.rs:1171-1245): per-sub-block min/max,
// 6-bit scales against d = max_scale/63 and dmin = max_min/63 (stored with
// the truncating f32->f16 above), then round((x + min)/scale) per element.
void quantize_q4k_block(const float *x, uint8_t *out) {
  float scale[8], negmin[8];
  for (int sb = 0; sb < 8; ++sb) {
    float lo = INFINITY, hi = -INFINITY;
    for (int i = 0; i < 32; ++i) {
      const float v = x[32 * sb + i];
      if (v < lo) lo = v;
      if (v > hi) hi = v;
    }
    if (lo >= 0.0f) {
      negmin[sb] = -0.0f;  // sub_mins = 0.0; the negated value enters only max() and rounding
      scale[sb] = hi > 0.0f ? hi / 15.0f : 0.0f;
    } else {
      negmin[sb] = -lo;
      scale[sb] = hi > lo ? (hi - lo) / 15.0f : 0.0f;
    }
  }
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; ++j) max_scale = std::fmax(max_scale, scale[j]), max_min = std::fmax(max_min, negmin[j]);
  const float d = max_scale > 0.0f ? max_scale / 63.0f : 0.0f;
  const float dmin = max_min > 0.0f ? max_min / 63.0f : 0.0f;
  uint8_t sv[8] = {}, mv[8] = {};
  if (d > 0.0f) {
    const float inv = 1.0f / d;
    for (int j = 0; j < 8; ++j) sv[j] = std::min<uint8_t>(sat_u8(scale[j] * inv + 0.5f), 63);
  }
  if (dmin > 0.0f) {
    const float inv = 1.0f / dmin;
    for (int j = 0; j < 8; ++j) mv[j] = std::min<uint8_t>(sat_u8(negmin[j] * inv + 0.5f), 63);
  }
  const uint16_t dh = float_to_half_trunc(d), mh = float_to_half_trunc(dmin);
  out[0] = (uint8_t)dh, out[1] = (uint8_t)(dh >> 8), out[2] = (uint8_t)mh, out[3] = (uint8_t)(mh >> 8);
  for (int j = 0; j < 4; ++j) {  // pack_scales (autograd2.rs:1119-1132)
    out[4 + j] = (uint8_t)((sv[j] & 63) | ((sv[j + 4] & 0x30) << 2));
    out[8 + j] = (uint8_t)((mv[j] & 63) | ((mv[j + 4] & 0x30) << 2));
    out[12 + j] = (uint8_t)((sv[j + 4] & 15) | ((mv[j + 4] & 15) << 4));
  }
  const float dv = half_to_float(dh), mvf = half_to_float(mh);
  for (int c = 0; c < 4; ++c) {
    const float a1 = dv * (float)sv[2 * c], b1 = mvf * (float)mv[2 * c];
    const float a2 = dv * (float)sv[2 * c + 1], b2 = mvf * (float)mv[2 * c + 1];
    for (int l = 0; l < 32; ++l) {
      const uint8_t q1 = a1 > 0.0f ? std::min<uint8_t>(sat_u8((x[64 * c + l] + b1) / a1 + 0.5f), 15) : 0;
      const uint8_t q2 = a2 > 0.0f ? std::min<uint8_t>(sat_u8((x[64 * c + 32 + l] + b2) / a2 + 0.5f), 15) : 0;
      out[16 + 32 * c + l] = (uint8_t)(q1 | (q2 << 4));
    }
  }
}

// Runs fn(r0, r1) over row bands on the host's hardware threads.
template <class F>
void parallel_rows(size_t rows, F fn) {
  const size_t hw = std::max(1u, std::thread::hardware_concurrency());
  const size_t nt = std::min(hw, std::max<size_t>(1, rows / 16));
  if (nt <= 1) return fn(0, rows);
  std::vector<std::thread> th;
  const size_t per = (rows + nt - 1) / nt;
  for (size_t t = 0; t < nt; ++t) {
    const size_t r0 = t * per, r1 = std::min(rows, r0 + per);
    if (r0 < r1) th.emplace_back(fn, r0, r1);
  }
  for (auto &t : th) t.join();
}

// Decode n_elem elements of a block-quantised tensor (tail blocks clipped).
rt_status decode_to_f32(int32_t type, const uint8_t *src, uint64_t n_elem, float *dst) {
  if (type == RT_GGUF_F32) {
    std::memcpy(dst, src, n_elem * 4);
    return RT_OK;
  }
  if (type == RT_GGUF_F16) {
    for (uint64_t i = 0; i < n_elem; ++i) dst[i] = half_to_float(le16(src + 2 * i));
    return RT_OK;
  }
  void (*dec)(const uint8_t *, float *) = nullptr;
  uint64_t bpb = 0, epb = 0;
  switch (type) {
    case RT_GGUF_Q4_0: dec = dec_q4_0; break;
    case RT_GGUF_Q8_0: dec = dec_q8_0; break;
    case RT_GGUF_Q4_K: dec = dec_q4k; break;
    case RT_GGUF_Q5_K: dec = dec_q5k; break;
    case RT_GGUF_Q6_K: dec = dec_q6k; break;
    default: return set_error(RT_EINVAL, "gguf: type %d has no f32 decoding (tensor_to_f32, gguf_loader.rs:745-760)", type);
  }
  block_info(type, bpb, epb);
  const uint64_t nb = (n_elem + epb - 1) / epb;
  parallel_rows(nb, [&](size_t b0, size_t b1) {
    float tmp[256];
    for (size_t b = b0; b < b1; ++b) {
      const uint64_t e0 = b * epb, n = std::min<uint64_t>(epb, n_elem - e0);
      if (n == epb) dec(src + b * bpb, dst + e0);
      else {
        dec(src + b * bpb, tmp);
        std::memcpy(dst + e0, tmp, n * 4);
      }
    }
  });
  return RT_OK;
}

}  // namespace

struct rt_gguf {
  std::string path;
  int fd = -1;
  uint64_t file_size = 0, data_start = 0;
  std::unordered_map<std::string, MetaValue> meta;
  std::vector<std::string> keys;  // file order, first occurrence of each key
  int64_t n_meta = 0;
  std::vector<TensorEntry> tensors;
};

namespace {

const TensorEntry *entry(const rt_gguf *g, int64_t idx) {
  if (!g || idx < 0 || idx >= (int64_t)g->tensors.size()) return nullptr;
  return &g->tensors[(size_t)idx];
}

const MetaValue *meta(const rt_gguf *g, const char *key) {
  if (!g || !key) return nullptr;
  auto it = g->meta.find(key);
  return it == g->meta.end() ? nullptr : &it->second;
}

rt_status read_bytes(const rt_gguf *g, const TensorEntry &t, void *dst) {
  // every comparison is against the file size, so no sum can wrap
  const bool inside = t.n_bytes > 0 && t.offset <= g->file_size && g->data_start <= g->file_size - t.offset &&
                      t.n_bytes <= g->file_size - (g->data_start + t.offset);
  const uint64_t at = inside ? g->data_start + t.offset : t.offset;
  if (!inside)
    return set_error(RT_EINVAL, "gguf: tensor '%s' (%llu bytes at data offset %llu) lies outside the file",
                     t.name.c_str(), (unsigned long long)t.n_bytes, (unsigned long long)t.offset);
  uint8_t *d = static_cast<uint8_t *>(dst);
  uint64_t done = 0;
  while (done < t.n_bytes) {
    const ssize_t got = pread(g->fd, d + done, (size_t)std::min<uint64_t>(t.n_bytes - done, 1ull << 30),
                              (off_t)(at + done));
    if (got <= 0) return set_error(RT_EINVAL, "gguf: short read of tensor '%s'", t.name.c_str());
    done += (uint64_t)got;
  }
  return RT_OK;
}

// The loader's extern "C" entry points allocate host memory (std::vector,
// std::string, threads): no C++ exception may cross the C boundary.
template <class F>
rt_status guarded(const char *who, F body) {
  try {
    return body();
  } catch (const std::bad_alloc &) {
    return set_error(RT_ENOMEM, "%s: out of host memory", who);
  } catch (const std::exception &e) {
    return set_error(RT_EINVAL, "%s: %s", who, e.what());
  } catch (...) {
    return set_error(RT_EINVAL, "%s: unexpected exception", who);
  }
}

}  // namespace

extern "C" {

static rt_status gguf_open(const char *path, rt_gguf **out) {
  if (!path || !out) return set_error(RT_EINVAL, "rt_gguf_open: null pointer");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return set_error(RT_EINVAL, "rt_gguf_open: cannot open '%s': %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return set_error(RT_EINVAL, "rt_gguf_open: cannot stat '%s'", path);
  }
  rt_gguf *g = nullptr;
  try {
    g = new rt_gguf();
  } catch (...) {
    close(fd);
    throw;
  }
  g->path = path, g->fd = fd, g->file_size = (uint64_t)st.st_size;
  try {
  Reader r(fd, g->file_size);
  auto fail = [&](const char *what) {
    rt_status s = set_error(RT_EINVAL, "rt_gguf_open: %s: %s (at byte %llu)", path, what, (unsigned long long)r.pos());
    rt_gguf_close(g);
    return s;
  };
  char magic[4];
  uint32_t version;
  uint64_t n_tensors, n_kv;
  if (!r.read(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return fail("not a GGUF file");
  if (!r.get(version)) return fail("truncated header");
  if (version < 2 || version > 3) return fail("unsupported GGUF version (2 and 3 are read)");
  if (!r.get(n_tensors) || !r.get(n_kv)) return fail("truncated header");
  if (n_tensors > g->file_size || n_kv > g->file_size) return fail("tensor or metadata count exceeds the file size");
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key;
    uint32_t type;
    MetaValue v;
    if (!r.str(key) || !r.get(type) || !read_value(r, (int32_t)type, v, 0)) return fail("bad metadata entry");
    if (!g->meta.count(key)) g->keys.push_back(key);
    g->meta[key] = std::move(v);  // a repeated key keeps the last value, as HashMap::insert does
  }
  g->n_meta = (int64_t)g->meta.size();
  g->tensors.resize((size_t)n_tensors);
  for (auto &t : g->tensors) {
    uint32_t nd, type;
    if (!r.str(t.name) || !r.get(nd)) return fail("bad tensor entry");
    if (nd > 4) return fail("tensor with more than 4 dimensions");
    t.n_dims = (int32_t)nd;
    t.n_elem = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      uint64_t v;
      if (!r.get(v)) return fail("bad tensor entry");
      t.dims[d] = (int64_t)v;
      if (v != 0 && t.n_elem > (1ull << 62) / v) return fail("tensor size overflows");
      t.n_elem *= v;
    }
    if (!r.get(type) || !r.get(t.offset)) return fail("bad tensor entry");
    t.type = (int32_t)type;
    uint64_t bpb, epb;
    t.n_bytes = block_info(t.type, bpb, epb) ? (t.n_elem + epb - 1) / epb * bpb : 0;
    if (t.n_bytes > g->file_size) return fail("a tensor is larger than the file");
  }
  uint64_t align = 32;  // general.alignment when it is an integer (gguf_loader.rs:218-221)
  if (meta(g, "general.alignment")) {
    uint64_t v;
    if (rt_gguf_meta_u64(g, "general.alignment", &v) == RT_OK && v > 0) align = v;
  }
  g->data_start = (r.pos() + align - 1) / align * align;
  *out = g;
  return RT_OK;
  } catch (...) {
    rt_gguf_close(g);
    throw;
  }
}

rt_status rt_gguf_open(const char *path, rt_gguf **out) {
  return guarded("rt_gguf_open", [&] { return gguf_open(path, out); });
}

rt_status rt_gguf_close(rt_gguf *g) {
  if (!g) return RT_OK;
  if (g->fd >= 0) close(g->fd);
  delete g;
  return RT_OK;
}

int64_t rt_gguf_n_tensors(const rt_gguf *g) { return g ? (int64_t)g->tensors.size() : -1; }
int64_t rt_gguf_n_metadata(const rt_gguf *g) { return g ? g->n_meta : -1; }
uint64_t rt_gguf_data_start(const rt_gguf *g) { return g ? g->data_start : 0; }

rt_status rt_gguf_tensor_info(const rt_gguf *g, int64_t idx, rt_gguf_tensor *out) {
  const TensorEntry *t = entry(g, idx);
  if (!t || !out) return set_error(RT_EINVAL, "rt_gguf_tensor_info: bad handle or index %lld", (long long)idx);
  out->name = t->name.c_str();
  out->n_dims = t->n_dims;
  for (int d = 0; d < 4; ++d) out->dims[d] = d < t->n_dims ? t->dims[d] : 1;
  out->type = t->type;
  out->offset = t->offset;
  out->n_bytes = t->n_bytes;
  return RT_OK;
}

int64_t rt_gguf_find_tensor(const rt_gguf *g, const char *name) {
  if (!g || !name) return -1;
  for (size_t i = 0; i < g->tensors.size(); ++i)
    if (g->tensors[i].name == name) return (int64_t)i;
  return -1;
}

rt_status rt_gguf_meta_key(const rt_gguf *g, int64_t i, const char **key) {
  if (!g || !key || i < 0 || i >= (int64_t)g->keys.size())
    return set_error(RT_EINVAL, "rt_gguf_meta_key: bad handle or index %lld", (long long)i);
  *key = g->keys[(size_t)i].c_str();
  return RT_OK;
}

rt_status rt_gguf_meta_type(const rt_gguf *g, const char *key, int32_t *type, int32_t *elem_type, uint64_t *count) {
  const MetaValue *v = meta(g, key);
  if (!v) return set_error(RT_EINVAL, "gguf: no metadata key '%s'", key ? key : "(null)");
  if (type) *type = v->type;
  if (elem_type) *elem_type = v->elem_type;
  if (count) *count = v->type == RT_GGUF_META_ARRAY ? (uint64_t)v->arr.size() : 1;
  return RT_OK;
}

rt_status rt_gguf_meta_u64(const rt_gguf *g, const char *key, uint64_t *out) {
  const MetaValue *v = meta(g, key);
  if (!v || !out) return set_error(RT_EINVAL, "gguf: no metadata key '%s'", key ? key : "(null)");
  switch (v->type) {
    case RT_GGUF_META_U8: case RT_GGUF_META_U16: case RT_GGUF_META_U32: case RT_GGUF_META_U64:
      *out = v->u; return RT_OK;
    case RT_GGUF_META_I32: case RT_GGUF_META_I64:
      *out = (uint64_t)v->i; return RT_OK;  // `as u64`, wrapping like the reference
    default:
      return set_error(RT_EINVAL, "gguf: metadata '%s' is not an unsigned/i32/i64 integer", key);
  }
}

rt_status rt_gguf_meta_f32(const rt_gguf *g, const char *key, float *out) {
  const MetaValue *v = meta(g, key);
  if (!v || !out) return set_error(RT_EINVAL, "gguf: no metadata key '%s'", key ? key : "(null)");
  if (v->type != RT_GGUF_META_F32 && v->type != RT_GGUF_META_F64)
    return set_error(RT_EINVAL, "gguf: metadata '%s' is not a float", key);
  *out = (float)v->f;
  return RT_OK;
}

rt_status rt_gguf_meta_str(const rt_gguf *g, const char *key, const char **out) {
  const MetaValue *v = meta(g, key);
  if (!v || !out) return set_error(RT_EINVAL, "gguf: no metadata key '%s'", key ? key : "(null)");
  if (v->type != RT_GGUF_META_STR) return set_error(RT_EINVAL, "gguf: metadata '%s' is not a string", key);
  *out = v->s.c_str();
  return RT_OK;
}

rt_status rt_gguf_meta_array_str(const rt_gguf *g, const char *key, uint64_t i, const char **out) {
  const MetaValue *v = meta(g, key);
  if (!v || !out) return set_error(RT_EINVAL, "gguf: no metadata key '%s'", key ? key : "(null)");
  if (v->type != RT_GGUF_META_ARRAY || v->elem_type != RT_GGUF_META_STR)
    return set_error(RT_EINVAL, "gguf: metadata '%s' is not a string array", key);
  if (i >= v->arr.size()) return set_error(RT_EINVAL, "gguf: index %llu beyond '%s'", (unsigned long long)i, key);
  *out = v->arr[(size_t)i].s.c_str();
  return RT_OK;
}

rt_status rt_gguf_read_tensor(const rt_gguf *g, int64_t idx, void *dst, uint64_t capacity) {
  const TensorEntry *t = entry(g, idx);
  if (!t || !dst) return set_error(RT_EINVAL, "rt_gguf_read_tensor: bad handle, index or buffer");
  if (t->n_bytes == 0)
    return set_error(RT_EINVAL, "rt_gguf_read_tensor: unsupported type %d for tensor '%s'", t->type, t->name.c_str());
  if (capacity < t->n_bytes)
    return set_error(RT_EINVAL, "rt_gguf_read_tensor: '%s' needs %llu bytes, buffer has %llu", t->name.c_str(),
                     (unsigned long long)t->n_bytes, (unsigned long long)capacity);
  return read_bytes(g, *t, dst);
}

static rt_status gguf_tensor_to_f32(const rt_gguf *g, int64_t idx, float *dst, uint64_t n_elem) {
  const TensorEntry *t = entry(g, idx);
  if (!t || !dst) return set_error(RT_EINVAL, "rt_gguf_tensor_to_f32: bad handle, index or buffer");
  if (n_elem < t->n_elem)
    return set_error(RT_EINVAL, "rt_gguf_tensor_to_f32: '%s' has %llu elements, buffer %llu", t->name.c_str(),
                     (unsigned long long)t->n_elem, (unsigned long long)n_elem);
  if (t->type == RT_GGUF_BF16 || t->n_bytes == 0)
    return set_error(RT_EINVAL, "gguf: tensor '%s' has unsupported type %d for f32 decoding", t->name.c_str(), t->type);
  std::vector<uint8_t> raw((size_t)t->n_bytes);
  rt_status s = read_bytes(g, *t, raw.data());
  if (s != RT_OK) return s;
  return decode_to_f32(t->type, raw.data(), t->n_elem, dst);
}

rt_status rt_gguf_tensor_to_f32(const rt_gguf *g, int64_t idx, float *dst, uint64_t n_elem) {
  return guarded("rt_gguf_tensor_to_f32", [&] { return gguf_tensor_to_f32(g, idx, dst, n_elem); });
}

static rt_status q4k_quantize(const float *src, size_t rows, size_t cols, uint8_t *blocks) {
  if (!src || !blocks) return set_error(RT_EINVAL, "rt_q4k_quantize: null pointer");
  if (cols == 0 || cols % 256 != 0)
    return set_error(RT_EINVAL, "rt_q4k_quantize: cols must be a multiple of 256, got %zu", cols);
  const size_t nb = cols / 256;
  parallel_rows(rows, [&](size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r)
      for (size_t b = 0; b < nb; ++b) quantize_q4k_block(src + r * cols + 256 * b, blocks + (r * nb + b) * 144);
  });
  return RT_OK;
}

rt_status rt_q4k_quantize(const float *src, size_t rows, size_t cols, uint8_t *blocks) {
  return guarded("rt_q4k_quantize", [&] { return q4k_quantize(src, rows, cols, blocks); });
}

// Q4KMat::quantize_from_bf16 (autograd2.rs:1252-1289): each row widened to
// f32 in a per-thread row buffer, then quantized block by block as above.
static rt_status q4k_quantize_bf16(const uint16_t *src, size_t rows, size_t cols, uint8_t *blocks) {
  if (!src || !blocks) return set_error(RT_EINVAL, "rt_q4k_quantize_bf16: null pointer");
  if (cols == 0 || cols % 256 != 0)
    return set_error(RT_EINVAL, "rt_q4k_quantize_bf16: cols must be a multiple of 256, got %zu", cols);
  const size_t nb = cols / 256;
  parallel_rows(rows, [&](size_t r0, size_t r1) {
    std::vector<float> row(cols);
    for (size_t r = r0; r < r1; ++r) {
      for (size_t c = 0; c < cols; ++c) {
        const uint32_t bits = (uint32_t)src[r * cols + c] << 16;
        std::memcpy(&row[c], &bits, 4);
      }
      for (size_t b = 0; b < nb; ++b) quantize_q4k_block(row.data() + 256 * b, blocks + (r * nb + b) * 144);
    }
  });
  return RT_OK;
}

rt_status rt_q4k_quantize_bf16(const uint16_t *src, size_t rows, size_t cols, uint8_t *blocks) {
  return guarded("rt_q4k_quantize_bf16", [&] { return q4k_quantize_bf16(src, rows, cols, blocks); });
}

static rt_status gguf_load_linear(const rt_gguf *g, int64_t idx, int32_t flags, rt_linear *out) {
  const TensorEntry *t = entry(g, idx);
  if (!t || !out) return set_error(RT_EINVAL, "rt_gguf_load_linear: bad handle or index");
  std::memset(out, 0, sizeof *out);
  if (t->n_dims < 1) return set_error(RT_EINVAL, "rt_gguf_load_linear: '%s' has no dimensions", t->name.c_str());
  // GGUF [in, out] -> [rows=out, cols=in] (transformer4.rs:1189-1194)
  const int64_t rows = t->n_dims >= 2 ? t->dims[1] : 1, cols = t->dims[0];
  std::vector<uint8_t> host;
  int32_t format = 0;
  switch (t->type) {
    case RT_GGUF_Q4_K: {  // decode_q4k_to_q4kmat (gguf_loader.rs:360-381): the bytes as they are
      if (cols % 256 != 0)
        return set_error(RT_EINVAL, "rt_gguf_load_linear: Q4_K tensor '%s' has %lld columns (needs a multiple of 256)",
                         t->name.c_str(), (long long)cols);
      host.resize((size_t)t->n_bytes);
      rt_status s = read_bytes(g, *t, host.data());
      if (s != RT_OK) return s;
      format = RT_LINEAR_Q4K;
      break;
    }
    case RT_GGUF_Q4_0: {  // Q4_0 -> Q4_K (transformer4.rs:1198-1207, autograd2.rs:1291-1320)
      if (cols % 256 != 0)
        return set_error(RT_EINVAL, "rt_gguf_load_linear: Q4_0 tensor '%s' has %lld columns (Q4_K needs a multiple of 256)",
                         t->name.c_str(), (long long)cols);
      std::vector<uint8_t> raw((size_t)t->n_bytes);
      rt_status s = read_bytes(g, *t, raw.data());
      if (s != RT_OK) return s;
      const size_t nb = (size_t)cols / 256;
      host.resize((size_t)rows * nb * 144);
      parallel_rows((size_t)rows, [&](size_t r0, size_t r1) {
        std::vector<float> row((size_t)cols);
        for (size_t r = r0; r < r1; ++r) {
          // rows start on 32-element block boundaries (cols % 256 == 0)
          for (size_t b = 0; b < (size_t)cols / 32; ++b) dec_q4_0(raw.data() + (r * (size_t)cols / 32 + b) * 18, row.data() + 32 * b);
          for (size_t b = 0; b < nb; ++b) quantize_q4k_block(row.data() + 256 * b, host.data() + (r * nb + b) * 144);
        }
      });
      format = RT_LINEAR_Q4K;
      break;
    }
    case RT_GGUF_BF16:
      host.resize((size_t)t->n_bytes);
      if (rt_status s = read_bytes(g, *t, host.data()); s != RT_OK) return s;
      format = RT_LINEAR_BF16;
      break;
    case RT_GGUF_F32:
      host.resize((size_t)t->n_bytes);
      if (rt_status s = read_bytes(g, *t, host.data()); s != RT_OK) return s;
      format = RT_LINEAR_F32;
      break;
    case RT_GGUF_Q6_K:
    case RT_GGUF_Q8_0:
      if ((flags & RT_LOAD_KEEP_PACKED) && cols % (t->type == RT_GGUF_Q6_K ? 256 : 32) == 0) {
        // packed in the planar device layout (rows start on block boundaries)
        std::vector<uint8_t> raw((size_t)t->n_bytes);
        if (rt_status s = read_bytes(g, *t, raw.data()); s != RT_OK) return s;
        host.resize(raw.size());
        if (t->type == RT_GGUF_Q6_K) {
          rt::q6k_repack_host(raw.data(), raw.size() / 210, host.data());
          format = RT_LINEAR_Q6K;
        } else {
          rt::q8_0_repack_host(raw.data(), raw.size() / 34, host.data());
          format = RT_LINEAR_Q8_0;
        }
        break;
      }
      [[fallthrough]];
    case RT_GGUF_F16: case RT_GGUF_Q5_K: {
      // widen to f32, then f32s_to_bf16_and_drop (transformer4.rs:1084-1097)
      std::vector<float> f((size_t)t->n_elem);
      rt_status s = rt_gguf_tensor_to_f32(g, idx, f.data(), t->n_elem);
      if (s != RT_OK) return s;
      host.resize((size_t)t->n_elem * 2);
      uint16_t *h = reinterpret_cast<uint16_t *>(host.data());
      for (size_t i = 0; i < f.size(); ++i) h[i] = float_to_bf16(f[i]);
      format = RT_LINEAR_BF16;
      break;
    }
    default:
      return set_error(RT_EINVAL, "rt_gguf_load_linear: unsupported type %d for tensor '%s'", t->type, t->name.c_str());
  }
  void *dev = nullptr;
  hipError_t e = hipMalloc(&dev, host.size());
  if (e != hipSuccess) return rt::hip_error(e, "rt_gguf_load_linear hipMalloc");
  e = hipMemcpy(dev, host.data(), host.size(), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(dev);
    return rt::hip_error(e, "rt_gguf_load_linear hipMemcpy");
  }
  out->format = format, out->src_type = t->type, out->rows = rows, out->cols = cols;
  out->data = dev, out->bytes = host.size();
  return RT_OK;
}

rt_status rt_gguf_load_linear_ex(const rt_gguf *g, int64_t idx, int32_t flags, rt_linear *out) {
  return guarded("rt_gguf_load_linear", [&] { return gguf_load_linear(g, idx, flags, out); });
}

rt_status rt_gguf_load_linear(const rt_gguf *g, int64_t idx, rt_linear *out) {
  return rt_gguf_load_linear_ex(g, idx, 0, out);
}

rt_status rt_linear_free(rt_linear *l) {
  if (!l) return RT_OK;
  if (l->data) {
    hipError_t e = hipFree(l->data);
    l->data = nullptr;
    if (e != hipSuccess) return rt::hip_error(e, "rt_linear_free");
  }
  return RT_OK;
}

}  // extern "C"
