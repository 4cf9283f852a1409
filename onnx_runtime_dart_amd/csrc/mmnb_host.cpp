// Host-only input handling of libmmnb: the ONNX wire reader and pack
// planner (for mmnb_model_load) and the MatMulNBits host preparation (for
// mmnb_pack_nbits_ex).  Built with the C++ host compiler into the library,
// and with g++ -fsanitize=address,undefined into the CPU fuzz harness.
#include "mmnb_host.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>

namespace mmnb {

// ===================================================== MatMulNBits (host)

float half_to_float(uint16_t h) {
  // subnormals m * 2^-24, normals (1024 + m) * 2^(e - 25), e = 31 inf / NaN
  const int sign = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = std::ldexp((float)m, -24);
  else if (e == 31) v = m ? std::nanf("") : INFINITY;
  else v = std::ldexp((float)(1024 + m), e - 25);
  return sign ? -v : v;
}

namespace {

// `need` values of type `type` from p, which holds len values of that type.
int read_floats(const void *p, int64_t len, int type, int64_t need, const char *what,
                std::vector<float> *out) {
  if (type != MMNB_DT_F32 && type != MMNB_DT_F16)
    return fail(MMNB_ERR_UNSUPPORTED, std::string("MatMulNBits: ") + what +
                                          " must be float32 or float16");
  if (!p || len < need)
    return fail(MMNB_ERR_ARG, std::string("MatMulNBits: ") + what + " has " +
                                  std::to_string(p ? len : 0) + " values, need " +
                                  std::to_string(need));
  out->resize((size_t)need);
  if (type == MMNB_DT_F32) {
    std::memcpy(out->data(), p, (size_t)need * 4);
  } else {
    const uint8_t *h = (const uint8_t *)p;
    for (int64_t i = 0; i < need; i++) {
      uint16_t v;
      std::memcpy(&v, h + 2 * i, 2);
      (*out)[(size_t)i] = half_to_float(v);
    }
  }
  return MMNB_OK;
}

}  // namespace

int nbits_prepare(const mmnb_nbits_desc *d, NbitsHost *out) {
  if (!d || !out) return fail(MMNB_ERR_ARG, "mmnb_pack_nbits_ex: null argument");
  const int64_t k = d->k, n = d->n, bits = d->bits, bs = d->block_size;
  if (bits != 4 && bits != 8)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: bits must be 4 or 8, got " + std::to_string(bits));
  if (k <= 0 || n <= 0) return fail(MMNB_ERR_ARG, "MatMulNBits: K and N must be positive");
  if (k > INT32_MAX / 2 || n > INT32_MAX)
    return fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: K or N too large for the kernels");
  // any even block size for the reference's own form (bits 4, uint8 zero
  // points, no g_idx / bias); the extensions need a power of two >= 16
  if (bs < 2 || (bs & 1) || bs > (int64_t(1) << 30))
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: block_size must be even and at most 2^30, got " +
                    std::to_string(bs));
  const bool native_block = bs >= 16 && (bs & (bs - 1)) == 0;
  if (bits == 8 && !native_block)
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: bits=8 needs a power-of-two block_size >= 16");
  const int64_t nb = (k + bs - 1) / bs;
  const int64_t blob = bs * bits / 8;
  int64_t nnb, need_b;
  if (!mul_nonneg(n, nb, &nnb) || !mul_nonneg(nnb, blob, &need_b))
    return fail(MMNB_ERR_ARG, "MatMulNBits: N * K too large");
  if (!d->b_q || d->b_q_len < need_b)
    return fail(MMNB_ERR_ARG, "MatMulNBits: B has " + std::to_string(d->b_q_len) +
                                  " bytes, need " + std::to_string(need_b));
  out->k = k;
  out->n = n;
  out->block = bs;
  out->n_blocks = nb;
  int rc;
  std::vector<float> s;
  if ((rc = read_floats(d->scales, d->scales_len, d->scales_type, nnb, "scales", &s))) return rc;
  // ---- zero points: integers (zi) or floats (zf), one per (column, block)
  std::vector<int32_t> zi;
  std::vector<float> zf;
  if (d->zero_points) {
    if (d->zero_points_type == MMNB_DT_U8) {
      const uint8_t *z = (const uint8_t *)d->zero_points;
      if (bits == 8) {
        if (d->zero_points_len < nnb)
          return fail(MMNB_ERR_ARG, "MatMulNBits: zero_points needs N*n_blocks bytes");
        zi.resize((size_t)nnb);
        for (int64_t i = 0; i < nnb; i++) zi[(size_t)i] = z[i];
      } else if (d->zero_points_layout == MMNB_ZP_PER_COLUMN) {
        const int64_t row = (nb + 1) / 2;
        if (d->zero_points_len / row < n)
          return fail(MMNB_ERR_ARG, "MatMulNBits: zero_points needs N*ceil(n_blocks/2) bytes");
        zi.resize((size_t)nnb);
        for (int64_t c = 0; c < n; c++)
          for (int64_t b = 0; b < nb; b++) {
            const uint8_t byte = z[c * row + b / 2];
            zi[(size_t)(c * nb + b)] = (b & 1) ? byte >> 4 : byte & 15;
          }
      } else if (d->zero_points_layout == MMNB_ZP_FLAT) {
        if (d->zero_points_len < (nnb + 1) / 2)
          return fail(MMNB_ERR_ARG, "MatMulNBits: zero_points needs ceil(N*n_blocks/2) bytes");
        zi.resize((size_t)nnb);
        for (int64_t i = 0; i < nnb; i++) {
          const uint8_t byte = z[i >> 1];
          zi[(size_t)i] = (i & 1) ? byte >> 4 : byte & 15;
        }
      } else {
        return fail(MMNB_ERR_ARG, "MatMulNBits: unknown zero-point layout");
      }
    } else if ((rc = read_floats(d->zero_points, d->zero_points_len, d->zero_points_type, nnb,
                                 "zero_points", &zf))) {
      return rc;
    }
  }
  if (d->bias && (rc = read_floats(d->bias, d->bias_len, d->bias_type, n, "bias", &out->bias)))
    return rc;
  // ---- g_idx: a stable sort of the rows by group, unless it is k / bs
  std::vector<int32_t> perm;
  if (d->g_idx) {
    if (d->g_idx_len != k) return fail(MMNB_ERR_ARG, "MatMulNBits: g_idx needs K entries");
    bool trivial = true;
    std::vector<int64_t> count((size_t)nb, 0);
    for (int64_t i = 0; i < k; i++) {
      const int32_t g = d->g_idx[i];
      if (g < 0 || g >= nb) return fail(MMNB_ERR_ARG, "MatMulNBits: g_idx out of range");
      count[(size_t)g]++;
      trivial = trivial && g == i / bs;
    }
    if (!trivial) {
      if (bits != 4)
        return fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: g_idx with bits=8 is not supported");
      if (k % bs)
        return fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: g_idx needs K a multiple of block_size");
      for (int64_t g = 0; g < nb; g++)
        if (count[(size_t)g] != bs)
          return fail(MMNB_ERR_UNSUPPORTED,
                      "MatMulNBits: g_idx groups must hold block_size rows each");
      perm.resize((size_t)k);
      for (int64_t i = 0; i < k; i++) perm[(size_t)i] = (int32_t)i;
      std::stable_sort(perm.begin(), perm.end(), [&](int32_t a, int32_t b) {
        return d->g_idx[a] < d->g_idx[b];
      });
    }
  }
  if (!native_block && (!zf.empty() || !out->bias.empty() || !perm.empty()))
    return fail(MMNB_ERR_UNSUPPORTED,
                "MatMulNBits: g_idx, bias and float zero points need a power-of-two "
                "block_size >= 16");
  // ---- the virtual 4-bit weight
  const uint8_t *B = d->b_q;
  const int64_t kp = nb * bs;
  const int64_t kv = bits == 8 ? 2 * kp : k;
  const int64_t nbv = (kv + bs - 1) / bs;
  const int64_t vblob = bs / 2;
  int64_t vbytes;
  if (!mul_nonneg(n * nbv, vblob, &vbytes))
    return fail(MMNB_ERR_ARG, "MatMulNBits: N * K too large");
  out->kv = kv;
  auto &vb = out->vb;
  auto &vs = out->vs;
  vs = s;
  auto nib4 = [&](int64_t c, int64_t kk) -> int {  // 4-bit q of column c, row kk
    const uint8_t byte = B[c * nb * blob + (kk / bs) * blob + (kk % bs) / 2];
    return (kk & 1) ? byte >> 4 : byte & 15;
  };
  auto put = [&](int64_t c, int64_t j, int q) {
    uint8_t &byte = vb[(size_t)(c * nbv * vblob + (j / bs) * vblob + (j % bs) / 2)];
    byte = (j & 1) ? (uint8_t)((byte & 0x0F) | (q << 4)) : (uint8_t)((byte & 0xF0) | q);
  };
  if (bits == 8) {
    vb.assign((size_t)vbytes, 0x88);
    for (int64_t c = 0; c < n; c++)
      for (int64_t kk = 0; kk < k; kk++) {
        const int q8 = B[c * nb * bs + kk];
        put(c, kk, q8 >> 4);
        put(c, kp + kk, q8 & 15);
      }
    vs.resize((size_t)(n * nbv));
    for (int64_t c = 0; c < n; c++)
      for (int64_t b = 0; b < nb; b++) {
        vs[(size_t)(c * nbv + b)] = 16.0f * s[(size_t)(c * nb + b)];
        vs[(size_t)(c * nbv + nb + b)] = s[(size_t)(c * nb + b)];
      }
    out->corr.assign((size_t)nnb, 0.0);
    for (int64_t c = 0; c < n; c++)
      for (int64_t b = 0; b < nb; b++) {
        const double z = !zf.empty() ? (double)zf[(size_t)(c * nb + b)]
                                     : !zi.empty() ? (double)zi[(size_t)(c * nb + b)] : 128.0;
        out->corr[(size_t)(b * n + c)] = (136.0 - z) * (double)s[(size_t)(c * nb + b)];
      }
    out->asrc.resize((size_t)kv);
    for (int64_t j = 0; j < kv; j++) {
      const int64_t kk = j < kp ? j : j - kp;
      out->asrc[(size_t)j] = kk < k ? (int32_t)kk : -1;
    }
  } else {
    if (perm.empty()) {
      vb.assign(B, B + need_b);
    } else {
      vb.assign((size_t)vbytes, 0);
      for (int64_t c = 0; c < n; c++)
        for (int64_t j = 0; j < k; j++) put(c, j, nib4(c, perm[(size_t)j]));
      out->asrc = perm;
    }
    if (!zf.empty()) {
      out->zfill = 0x00;  // the kernels see zero point 0; -z s goes to the correction
      out->corr.assign((size_t)nnb, 0.0);
      for (int64_t c = 0; c < n; c++)
        for (int64_t b = 0; b < nb; b++)
          out->corr[(size_t)(b * n + c)] =
              -(double)zf[(size_t)(c * nb + b)] * (double)s[(size_t)(c * nb + b)];
    } else if (!zi.empty()) {
      out->vz.assign((size_t)((nnb + 1) / 2), 0);
      for (int64_t i = 0; i < nnb; i++)
        out->vz[(size_t)(i >> 1)] |= (uint8_t)(zi[(size_t)i] << ((i & 1) * 4));
    }
  }
  return MMNB_OK;
}

namespace onnx {

// ============================================================ wire format
// A key varint (field << 3 | wire type) then a varint (0), a fixed64 (1), a
// length-delimited run (2) or a fixed32 (5).
namespace {

struct Field {
  uint32_t no = 0;
  int wt = 0;
  uint64_t v = 0;  // varint / fixed value (wire types 0, 1, 5)
  Span s;          // payload (wire type 2)
};

class Reader {
 public:
  explicit Reader(Span s) : p_(s.p), end_(s.p + s.n) {}
  // The next field; false at the end or (with *bad set) on malformed bytes.
  bool next(Field *f, bool *bad) {
    if (p_ >= end_) return false;
    uint64_t key;
    if (!varint(&key) || (key >> 3) == 0 || (key >> 3) > 0x1FFFFFFF) return fail_(bad);
    *f = Field();
    f->no = (uint32_t)(key >> 3);
    f->wt = (int)(key & 7);
    switch (f->wt) {
      case 0:
        if (!varint(&f->v)) return fail_(bad);
        return true;
      case 1:
        if (end_ - p_ < 8) return fail_(bad);
        std::memcpy(&f->v, p_, 8);
        p_ += 8;
        return true;
      case 2: {
        uint64_t len;
        if (!varint(&len) || len > (uint64_t)(end_ - p_)) return fail_(bad);
        f->s = Span{p_, (size_t)len};
        p_ += len;
        return true;
      }
      case 5: {
        if (end_ - p_ < 4) return fail_(bad);
        uint32_t v;
        std::memcpy(&v, p_, 4);
        f->v = v;
        p_ += 4;
        return true;
      }
      default:
        return fail_(bad);
    }
  }
  bool done() const { return p_ >= end_; }
  bool varint(uint64_t *out) {
    uint64_t r = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (p_ >= end_) return false;
      const uint8_t b = *p_++;
      r |= (uint64_t)(b & 0x7F) << shift;
      if (!(b & 0x80)) {
        *out = r;
        return true;
      }
    }
    return false;
  }

 private:
  static bool fail_(bool *bad) {
    *bad = true;
    return false;
  }
  const uint8_t *p_, *end_;
};

// Repeated scalar field: packed (one length-delimited run of varints) or not.
bool read_varints(const Field &f, std::vector<int64_t> *out) {
  if (f.wt == 0) {
    out->push_back((int64_t)f.v);
    return true;
  }
  if (f.wt != 2) return false;
  Reader r(f.s);
  uint64_t v;
  while (!r.done()) {
    if (!r.varint(&v)) return false;
    out->push_back((int64_t)v);
  }
  return true;
}

std::string str(const Span &s) { return std::string((const char *)s.p, s.n); }

// ONNX TensorProto.DataType codes handled for weights.
enum { kF32 = 1, kU8 = 2, kI8 = 3, kI32 = 6, kI64 = 7, kF16 = 10 };

int elem_size(int dt) {
  switch (dt) {
    case kF32: case kI32: return 4;
    case kU8: case kI8: return 1;
    case kI64: return 8;
    case kF16: return 2;
    default: return 0;
  }
}

struct Tensor {
  std::string name;
  int dtype = 0;
  std::vector<int64_t> dims;
  Span raw;                   // raw_data
  Span float_data;            // packed float_data
  std::vector<int64_t> ints;  // int32_data / int64_data
  bool has_raw = false, has_floats = false, has_ints = false;
  bool external = false;
  std::string location;
  int64_t offset = 0, length = 0;
  bool has_offset = false, has_length = false;
};

struct Node {
  std::string name, op, domain;
  std::vector<std::string> in, out;
  std::unordered_map<std::string, int64_t> ints;  // integer attributes
};

// A decimal int64 (the external_data offset / length values); false on
// anything else.
bool parse_i64(const std::string &s, int64_t *v) {
  if (s.empty() || s.size() > 19) return false;
  int64_t r = 0;
  for (char c : s) {
    if (c < '0' || c > '9') return false;
    r = r * 10 + (c - '0');
  }
  *v = r;
  return true;
}

// TensorProto (onnx.proto3): dims = 1, data_type = 2, float_data = 4,
// int32_data = 5, name = 8, raw_data = 9, int64_data = 7,
// external_data = 13 (StringStringEntryProto {key = 1, value = 2}),
// data_location = 14.  A field with the wrong wire type is malformed.
bool parse_tensor(Span s, Tensor *t) {
  Reader r(s);
  Field f;
  bool bad = false;
  while (r.next(&f, &bad)) {
    switch (f.no) {
      case 1:
        if (!read_varints(f, &t->dims)) return false;
        break;
      case 2:
        if (f.wt != 0) return false;
        t->dtype = f.v > INT_MAX ? -1 : (int)f.v;
        break;
      case 4:
        if (f.wt != 2) return false;  // unpacked float_data: not written by exporters
        t->float_data = f.s;
        t->has_floats = true;
        break;
      case 5: case 7:
        if (!read_varints(f, &t->ints)) return false;
        t->has_ints = true;
        break;
      case 8:
        if (f.wt != 2) return false;
        t->name = str(f.s);
        break;
      case 9:
        if (f.wt != 2) return false;
        t->raw = f.s;
        t->has_raw = true;
        break;
      case 13: {
        if (f.wt != 2) return false;
        Reader e(f.s);
        Field g;
        std::string key, val;
        while (e.next(&g, &bad)) {
          if (g.no != 1 && g.no != 2) continue;
          if (g.wt != 2) return false;
          (g.no == 1 ? key : val) = str(g.s);
        }
        if (bad) return false;
        if (key == "location") {
          t->location = val;
        } else if (key == "offset") {
          if (!parse_i64(val, &t->offset)) return false;
          t->has_offset = true;
        } else if (key == "length") {
          if (!parse_i64(val, &t->length)) return false;
          t->has_length = true;
        }
        break;
      }
      case 14:
        if (f.wt != 0) return false;
        t->external = f.v == 1;
        break;
      default:
        break;
    }
  }
  return !bad;
}

// NodeProto: input = 1, output = 2, name = 3, op_type = 4, attribute = 5
// (AttributeProto {name = 1, i = 3}), domain = 7.
bool parse_node(Span s, Node *n) {
  Reader r(s);
  Field f;
  bool bad = false;
  while (r.next(&f, &bad)) {
    if (f.no >= 1 && f.no <= 7 && f.no != 6 && f.wt != 2) return false;
    switch (f.no) {
      case 1: n->in.push_back(str(f.s)); break;
      case 2: n->out.push_back(str(f.s)); break;
      case 3: n->name = str(f.s); break;
      case 4: n->op = str(f.s); break;
      case 7: n->domain = str(f.s); break;
      case 5: {
        Reader a(f.s);
        Field g;
        std::string an;
        int64_t iv = 0;
        bool has_i = false;
        while (a.next(&g, &bad)) {
          if (g.no == 1) {
            if (g.wt != 2) return false;
            an = str(g.s);
          } else if (g.no == 3) {
            if (g.wt != 0) return false;
            iv = (int64_t)g.v;
            has_i = true;
          }
        }
        if (bad) return false;
        if (has_i) n->ints[an] = iv;
        break;
      }
      default: break;
    }
  }
  return !bad;
}

bool count_of(const std::vector<int64_t> &dims, int64_t *out) {
  int64_t c = 1;
  for (int64_t d : dims)
    if (!mul_nonneg(c, d, &c)) return false;
  *out = c;
  return true;
}

// Tensor t's bytes (raw, external or inline), checked against its shape and
// element type.
int tensor_bytes(const Tensor &t, ExternalData *ext, WeightBytes *b) {
  b->dtype = t.dtype;
  b->dims = t.dims;
  for (int64_t d : t.dims)
    if (d < 0) return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" has a negative dimension");
  const int es = elem_size(t.dtype);
  if (!es)
    return fail(MMNB_ERR_UNSUPPORTED, "Unsupported ONNX TensorProto dataType " +
                                          std::to_string(t.dtype) + " for \"" + t.name + "\"");
  int64_t cnt, need;
  if (!count_of(t.dims, &cnt) || !mul_nonneg(cnt, es, &need))
    return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" is too large");
  b->count = cnt;
  if (t.external) {
    if (!ext) return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" has external data");
    int rc = check_ref(t.location, 0, 0, 0);  // path safety before touching disk
    if (rc) return rc;
    const int64_t len = t.has_length && t.length > 0 ? t.length : need;
    Span file;
    if ((rc = ext->get(t.location, &file))) return rc;
    if ((rc = check_ref(t.location, t.offset, len, (int64_t)file.n))) return rc;
    if (len < need) return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" external data too short");
    b->p = file.p + t.offset;
    b->n = (size_t)need;
    return MMNB_OK;
  }
  if (t.has_raw) {
    if ((int64_t)t.raw.n < need)
      return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" raw_data too short");
    b->p = t.raw.p;
    b->n = (size_t)need;
    return MMNB_OK;
  }
  if (t.has_floats && t.dtype == kF32) {
    if ((int64_t)t.float_data.n != need)
      return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" inline data length mismatch");
    b->p = t.float_data.p;
    b->n = (size_t)need;
    return MMNB_OK;
  }
  if (t.has_ints) {
    if ((int64_t)t.ints.size() != cnt)
      return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" inline data length mismatch");
    b->own.resize((size_t)need);
    for (int64_t i = 0; i < cnt; i++) {
      const int64_t v = t.ints[(size_t)i];
      uint8_t *dst = &b->own[(size_t)(i * es)];
      if (es == 1) {
        *dst = (uint8_t)v;
      } else if (es == 2) {
        const uint16_t h = (uint16_t)v;
        std::memcpy(dst, &h, 2);
      } else if (es == 4) {
        const int32_t w = (int32_t)v;
        std::memcpy(dst, &w, 4);
      } else {
        std::memcpy(dst, &v, 8);
      }
    }
    b->p = b->own.data();
    b->n = (size_t)need;
    return MMNB_OK;
  }
  if (cnt == 0) return MMNB_OK;
  return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" has no data");
}

int64_t attr(const Node &n, const char *name, int64_t dflt, bool *found = nullptr) {
  auto it = n.ints.find(name);
  if (found) *found = it != n.ints.end();
  return it != n.ints.end() ? it->second : dflt;
}

// MMNB_DT_F32 / MMNB_DT_F16 for a float initializer, 0 for any other type
// (a uint8 or int32 tensor is never reinterpreted as floats).
int dt_float(int dtype) { return dtype == kF16 ? MMNB_DT_F16 : dtype == kF32 ? MMNB_DT_F32 : 0; }

// Zero points of an integer op: a uint8/int8 tensor as int64 values.
int int_zero_points(const std::string &op, const WeightBytes &z, std::vector<int64_t> *out) {
  if (z.dtype != kU8 && z.dtype != kI8)
    return fail(MMNB_ERR_UNSUPPORTED, op + ": zero point must be uint8/int8");
  out->resize((size_t)z.count);
  for (size_t i = 0; i < out->size(); i++)
    (*out)[i] = z.dtype == kI8 ? (int64_t)(int8_t)z.p[i] : (int64_t)z.p[i];
  return MMNB_OK;
}

}  // namespace

int check_ref(const std::string &loc, int64_t off, int64_t len, int64_t file_len) {
  if (loc.empty() || loc.find("..") != std::string::npos || loc[0] == '/' || loc[0] == '\\' ||
      loc.find(':') != std::string::npos || loc.find('\0') != std::string::npos)
    return fail(MMNB_ERR_ARG, "unsafe external-data location: \"" + loc + "\"");
  if (off < 0 || len < 0 || len > file_len || off > file_len - len)
    return fail(MMNB_ERR_ARG, "external-data range [" + std::to_string(off) + ", +" +
                                  std::to_string(len) + ") lies outside the companion file (" +
                                  std::to_string(file_len) + " bytes)");
  return MMNB_OK;
}

MappedFile::~MappedFile() {
  if (base && len) munmap(base, len);
}

int map_file(const std::string &path, MappedFile *m) {
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) return fail(MMNB_ERR_ARG, "model: cannot open " + path);
  struct stat st;
  if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
    close(fd);
    return fail(MMNB_ERR_ARG, "model: not a regular file: " + path);
  }
  m->len = (size_t)st.st_size;
  if (m->len) {
    void *b = mmap(nullptr, m->len, PROT_READ, MAP_PRIVATE, fd, 0);
    if (b == MAP_FAILED) {
      m->len = 0;
      close(fd);
      return fail(MMNB_ERR_ARG, "model: cannot map " + path);
    }
    m->base = b;
  }
  close(fd);
  return MMNB_OK;
}

int MappedExternalData::get(const std::string &loc, Span *out) {
  auto it = maps_.find(loc);
  if (it == maps_.end()) {
    std::unique_ptr<MappedFile> m(new MappedFile());
    int rc = map_file(dir_ + "/" + loc, m.get());
    if (rc) return rc;
    it = maps_.emplace(loc, std::move(m)).first;
  }
  *out = it->second->span();
  return MMNB_OK;
}

int scan_model(Span model, ExternalData *ext, std::vector<PackPlan> *plans) {
  // ModelProto.graph = 7; GraphProto.node = 1, .initializer = 5
  Span graph;
  bool has_graph = false;
  {
    Reader r(model);
    Field f;
    bool bad = false;
    while (r.next(&f, &bad))
      if (f.no == 7) {
        if (f.wt != 2) return fail(MMNB_ERR_ARG, "model: malformed protobuf");
        graph = f.s;
        has_graph = true;
      }
    if (bad) return fail(MMNB_ERR_ARG, "model: malformed protobuf");
  }
  if (!has_graph) return fail(MMNB_ERR_ARG, "model: no graph");
  std::vector<Node> nodes;
  std::unordered_map<std::string, Tensor> inits;
  {
    Reader r(graph);
    Field f;
    bool bad = false;
    while (r.next(&f, &bad)) {
      if (f.no != 1 && f.no != 5) continue;
      if (f.wt != 2) return fail(MMNB_ERR_ARG, "model: malformed graph");
      if (f.no == 1) {
        Node n;
        if (!parse_node(f.s, &n)) return fail(MMNB_ERR_ARG, "model: malformed node");
        nodes.push_back(std::move(n));
      } else {
        Tensor t;
        if (!parse_tensor(f.s, &t)) return fail(MMNB_ERR_ARG, "model: malformed initializer");
        std::string name = t.name;
        inits[name] = std::move(t);
      }
    }
    if (bad) return fail(MMNB_ERR_ARG, "model: malformed graph");
  }
  auto init = [&](const Node &n, size_t i) -> const Tensor * {
    if (i >= n.in.size() || n.in[i].empty()) return nullptr;
    auto it = inits.find(n.in[i]);
    return it == inits.end() ? nullptr : &it->second;
  };
  auto given = [](const Node &n, size_t i) { return i < n.in.size() && !n.in[i].empty(); };
  int rc;
  for (const Node &n : nodes) {
    PackPlan pl;
    pl.op = n.op;
    pl.label = !n.name.empty() ? n.name : (n.out.empty() ? n.op : n.out[0]);
    if (n.op == "MatMulNBits") {
      const Tensor *tb = init(n, 1), *ts = init(n, 2), *tz = init(n, 3), *tg = init(n, 4),
                   *tbias = init(n, 5);
      if (!tb || !ts) continue;
      if ((given(n, 3) && !tz) || (given(n, 4) && !tg) || (given(n, 5) && !tbias))
        continue;  // a dynamic input
      pl.kind = kPlanNBits;
      mmnb_nbits_desc &d = pl.nbits;
      bool fk, fn, fbs;
      d.k = attr(n, "K", 0, &fk);
      d.n = attr(n, "N", 0, &fn);
      d.bits = attr(n, "bits", 4);
      d.block_size = attr(n, "block_size", 0, &fbs);
      if (!fk || !fn || !fbs)
        return fail(MMNB_ERR_ARG, "MatMulNBits " + pl.label + ": K, N, block_size required");
      pl.keep.resize(5);
      WeightBytes &bb = pl.keep[0], &bs = pl.keep[1], &bz = pl.keep[2], &bg = pl.keep[3],
                  &bbias = pl.keep[4];
      if ((rc = tensor_bytes(*tb, ext, &bb)) || (rc = tensor_bytes(*ts, ext, &bs))) return rc;
      if (tb->dtype != kU8) return fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: B must be uint8");
      d.b_q = bb.p;
      d.b_q_len = (int64_t)bb.n;
      d.scales = bs.p;
      d.scales_len = bs.count;
      d.scales_type = dt_float(ts->dtype);
      if (!d.scales_type)
        return fail(MMNB_ERR_UNSUPPORTED,
                    "MatMulNBits " + pl.label + ": scales must be float or float16");
      if (tz) {
        if ((rc = tensor_bytes(*tz, ext, &bz))) return rc;
        d.zero_points = bz.p;
        d.zero_points_len = bz.count;
        d.zero_points_type = tz->dtype == kU8 ? MMNB_DT_U8 : dt_float(tz->dtype);
        if (!d.zero_points_type)
          return fail(MMNB_ERR_UNSUPPORTED,
                      "MatMulNBits " + pl.label + ": zero points must be uint8, float or float16");
        d.zero_points_layout = tz->dims.size() == 2 ? MMNB_ZP_PER_COLUMN : MMNB_ZP_FLAT;
      }
      if (tg) {
        if ((rc = tensor_bytes(*tg, ext, &bg))) return rc;
        if (tg->dtype != kI32 && tg->dtype != kI64)
          return fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: g_idx must be int32 or int64");
        pl.g_idx.resize((size_t)bg.count);
        for (size_t i = 0; i < pl.g_idx.size(); i++) {
          int64_t v;
          if (tg->dtype == kI64) {
            std::memcpy(&v, bg.p + 8 * i, 8);
          } else {
            int32_t w;
            std::memcpy(&w, bg.p + 4 * i, 4);
            v = w;
          }
          if (v < INT32_MIN || v > INT32_MAX)
            return fail(MMNB_ERR_ARG, "MatMulNBits: g_idx out of range");
          pl.g_idx[i] = (int32_t)v;
        }
        d.g_idx = pl.g_idx.data();
        d.g_idx_len = (int64_t)pl.g_idx.size();
      }
      if (tbias) {
        if ((rc = tensor_bytes(*tbias, ext, &bbias))) return rc;
        d.bias = bbias.p;
        d.bias_len = bbias.count;
        d.bias_type = dt_float(tbias->dtype);
        if (!d.bias_type)
          return fail(MMNB_ERR_UNSUPPORTED,
                      "MatMulNBits " + pl.label + ": bias must be float or float16");
      }
    } else if (n.op == "MatMulInteger" || n.op == "QLinearMatMul") {
      const bool q = n.op == "QLinearMatMul";
      const size_t bi = q ? 3 : 1, zi = q ? 5 : 3;
      const Tensor *tb = init(n, bi), *tz = init(n, zi);
      if (!tb || (given(n, zi) && !tz)) continue;
      pl.kind = kPlanInteger;
      pl.keep.resize(2);
      WeightBytes &bb = pl.keep[0], &bz = pl.keep[1];
      if ((rc = tensor_bytes(*tb, ext, &bb))) return rc;
      if ((tb->dtype != kU8 && tb->dtype != kI8) || tb->dims.size() < 2)
        return fail(MMNB_ERR_UNSUPPORTED, n.op + ": B must be uint8/int8, rank >= 2");
      if (tz) {
        if ((rc = tensor_bytes(*tz, ext, &bz))) return rc;
        if ((rc = int_zero_points(n.op, bz, &pl.zero_point))) return rc;
      }
      pl.w = bb.p;
      pl.w_signed = tb->dtype == kI8;
      pl.k = tb->dims[tb->dims.size() - 2];
      pl.n = tb->dims.back();
      // w holds batch * k * n = count bytes; batch * n is bounded separately
      // for k = 0, where the count says nothing about it
      int64_t bn;
      if (!count_of(std::vector<int64_t>(tb->dims.begin(), tb->dims.end() - 2), &pl.batch) ||
          !mul_nonneg(pl.batch, pl.n, &bn) || bn > INT32_MAX || pl.k > INT32_MAX)
        return fail(MMNB_ERR_UNSUPPORTED, n.op + ": B is too large");
    } else if (n.op == "ConvInteger" || n.op == "QLinearConv") {
      const bool q = n.op == "QLinearConv";
      const size_t wi = q ? 3 : 1, zi = q ? 5 : 3;
      const Tensor *tw = init(n, wi), *tz = init(n, zi);
      if (!tw || (given(n, zi) && !tz)) continue;
      pl.kind = kPlanConv;
      pl.keep.resize(2);
      WeightBytes &bw = pl.keep[0], &bz = pl.keep[1];
      if ((rc = tensor_bytes(*tw, ext, &bw))) return rc;
      if (tw->dtype != kU8 && tw->dtype != kI8)
        return fail(MMNB_ERR_UNSUPPORTED, n.op + ": W must be uint8/int8");
      std::vector<int64_t> dims = tw->dims;
      if (dims.size() == 3) dims.insert(dims.begin() + 2, 1);  // 1-D as 2-D
      if (dims.size() != 4)
        return fail(MMNB_ERR_UNSUPPORTED, n.op + ": 1-D or 2-D convolutions only");
      if (tz) {
        if ((rc = tensor_bytes(*tz, ext, &bz))) return rc;
        if ((rc = int_zero_points(n.op, bz, &pl.zero_point))) return rc;
      }
      pl.w = bw.p;
      pl.w_signed = tw->dtype == kI8;
      pl.co = dims[0];
      pl.ci = dims[1];
      pl.kh = dims[2];
      pl.kw = dims[3];
      pl.group = attr(n, "group", 1);
    } else {
      continue;
    }
    plans->push_back(std::move(pl));
  }
  return MMNB_OK;
}

}  // namespace onnx
}  // namespace mmnb
