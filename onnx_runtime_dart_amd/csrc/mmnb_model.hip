// Weight-pack loader: the quantized weights of an ONNX model file go
// straight from the file to resident device packs.
//
// The reference parses the whole ModelProto into Dart tensors
// (lib/src/onnx_proto_loader.dart) and resolves external data with random
// access reads (lib/onnx_runtime_dart_io.dart:19-42); its quantized ops then
// take those host tensors on every call.  Here one call walks the graph's
// nodes, and for every MatMulNBits, MatMulInteger, QLinearMatMul,
// ConvInteger and QLinearConv whose weight inputs are initializers builds the
// device pack directly from the bytes: inline raw_data is read in place from
// the memory-mapped model, external data from the memory-mapped companion
// file (so a multi-GB file is never copied into host memory whole), and only
// small inline typed lists (int32_data / float_data) are decoded.  External
// references pass the reference's guard (checkExternalRef,
// onnx_runtime_dart_io.dart:44-69) and a missing/zero length falls back to
// the size the shape implies (onnx_proto_loader.dart:80-112).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "mmnb_internal.h"

using namespace mmnb;

namespace {

// ---------------------------------------------------------------- protobuf
// Wire format: a key varint (field << 3 | wire type) then a varint (0), a
// fixed64 (1), a length-delimited run (2) or a fixed32 (5).
struct Span {
  const uint8_t *p = nullptr;
  size_t n = 0;
};

struct Field {
  uint32_t no = 0;
  int wt = 0;
  uint64_t v = 0;  // varint / fixed value
  Span s;          // length-delimited payload
};

class Reader {
 public:
  explicit Reader(Span s) : p_(s.p), end_(s.p + s.n) {}
  bool next(Field *f, bool *bad) {
    if (p_ >= end_) return false;
    uint64_t key;
    if (!varint(&key) || (key >> 3) == 0 || (key >> 3) > 0x1FFFFFFF) return fail(bad);
    f->no = (uint32_t)(key >> 3);
    f->wt = (int)(key & 7);
    switch (f->wt) {
      case 0:
        if (!varint(&f->v)) return fail(bad);
        return true;
      case 1:
        if (end_ - p_ < 8) return fail(bad);
        std::memcpy(&f->v, p_, 8);
        p_ += 8;
        return true;
      case 2: {
        uint64_t len;
        if (!varint(&len) || len > (uint64_t)(end_ - p_)) return fail(bad);
        f->s = Span{p_, (size_t)len};
        p_ += len;
        return true;
      }
      case 5: {
        if (end_ - p_ < 4) return fail(bad);
        uint32_t v;
        std::memcpy(&v, p_, 4);
        f->v = v;
        p_ += 4;
        return true;
      }
      default:
        return fail(bad);
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
  static bool fail(bool *bad) {
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
  Span raw;                  // raw_data (into the mapped model)
  Span float_data;           // packed float_data
  std::vector<int64_t> ints; // int32_data / int64_data
  bool has_floats = false, has_ints = false;
  bool external = false;
  std::string location;
  int64_t offset = 0, length = 0;
};

struct Attr {
  int64_t i = 0;
  bool has_i = false;
};

struct Node {
  std::string name, op, domain;
  std::vector<std::string> in, out;
  std::unordered_map<std::string, Attr> attrs;
};

bool parse_tensor(Span s, Tensor *t) {
  Reader r(s);
  Field f;
  bool bad = false;
  while (r.next(&f, &bad)) {
    switch (f.no) {
      case 1:
        if (!read_varints(f, &t->dims)) return false;
        break;
      case 2: t->dtype = (int)f.v; break;
      case 4:
        if (f.wt == 2) {
          t->float_data = f.s;
          t->has_floats = true;
        } else if (f.wt == 5) {
          return false;  // unpacked float_data: not produced by exporters
        }
        break;
      case 5: case 7:
        if (!read_varints(f, &t->ints)) return false;
        t->has_ints = true;
        break;
      case 8: t->name = str(f.s); break;
      case 9: t->raw = f.s; break;
      case 13: {  // external_data: StringStringEntryProto {key = 1, value = 2}
        Reader e(f.s);
        Field g;
        std::string key, val;
        while (e.next(&g, &bad))
          if (g.no == 1) key = str(g.s);
          else if (g.no == 2) val = str(g.s);
        if (key == "location") t->location = val;
        else if (key == "offset") t->offset = std::strtoll(val.c_str(), nullptr, 10);
        else if (key == "length") t->length = std::strtoll(val.c_str(), nullptr, 10);
        break;
      }
      case 14: t->external = f.v == 1; break;
      default: break;
    }
  }
  return !bad;
}

bool parse_node(Span s, Node *n) {
  Reader r(s);
  Field f;
  bool bad = false;
  while (r.next(&f, &bad)) {
    switch (f.no) {
      case 1: n->in.push_back(str(f.s)); break;
      case 2: n->out.push_back(str(f.s)); break;
      case 3: n->name = str(f.s); break;
      case 4: n->op = str(f.s); break;
      case 7: n->domain = str(f.s); break;
      case 5: {  // AttributeProto {name = 1, i = 3}
        Reader a(f.s);
        Field g;
        std::string an;
        Attr at;
        while (a.next(&g, &bad))
          if (g.no == 1) an = str(g.s);
          else if (g.no == 3) {
            at.i = (int64_t)g.v;
            at.has_i = true;
          }
        n->attrs[an] = at;
        break;
      }
      default: break;
    }
  }
  return !bad;
}

// ------------------------------------------------------------------- files
struct Mapping {
  void *base = nullptr;
  size_t len = 0;
  ~Mapping() {
    if (base && base != MAP_FAILED && len) munmap(base, len);
  }
};

int map_file(const std::string &path, Mapping *m) {
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) return fail(MMNB_ERR_ARG, "model: cannot open " + path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return fail(MMNB_ERR_ARG, "model: cannot stat " + path);
  }
  m->len = (size_t)st.st_size;
  if (m->len) {
    m->base = mmap(nullptr, m->len, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m->base == MAP_FAILED) {
      m->base = nullptr;
      close(fd);
      return fail(MMNB_ERR_ARG, "model: cannot map " + path);
    }
  }
  close(fd);
  return MMNB_OK;
}

// A weight's bytes: a span into a mapping, or decoded into `own`.
struct Bytes {
  const uint8_t *p = nullptr;
  size_t n = 0;
  std::vector<uint8_t> own;
  int dtype = 0;
  std::vector<int64_t> dims;
  int64_t count() const {
    int64_t c = 1;
    for (int64_t d : dims) c *= d;
    return c;
  }
};

}  // namespace

struct mmnb_model {
  mmnb_ctx *ctx = nullptr;
  struct Entry {
    std::string op, name;
    mmnb_pack *pack = nullptr;
  };
  std::vector<Entry> entries;
};

namespace {

int check_ref(const std::string &loc, int64_t off, int64_t len, int64_t file_len) {
  if (loc.empty() || loc.find("..") != std::string::npos || loc[0] == '/' || loc[0] == '\\' ||
      loc.find(':') != std::string::npos)
    return fail(MMNB_ERR_ARG, "unsafe external-data location: \"" + loc + "\"");
  if (off < 0 || len < 0 || len > file_len || off > file_len - len)
    return fail(MMNB_ERR_ARG, "external-data range [" + std::to_string(off) + ", +" +
                                  std::to_string(len) + ") lies outside the companion file (" +
                                  std::to_string(file_len) + " bytes)");
  return MMNB_OK;
}

class Loader {
 public:
  explicit Loader(const std::string &dir) : dir_(dir) {}

  // Resolves tensor t's bytes (raw, external or inline).
  int bytes(const Tensor &t, Bytes *b) {
    b->dtype = t.dtype;
    b->dims = t.dims;
    for (int64_t d : t.dims)
      if (d < 0) return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" has a negative dimension");
    const int es = elem_size(t.dtype);
    if (!es)
      return fail(MMNB_ERR_UNSUPPORTED,
                  "Unsupported ONNX TensorProto dataType " + std::to_string(t.dtype) +
                      " for \"" + t.name + "\"");
    const int64_t cnt = b->count();
    const int64_t need = cnt * es;
    if (t.external) {
      const int64_t len = t.length > 0 ? t.length : need;
      Mapping *m = nullptr;
      int rc = ext(t.location, &m);
      if (rc) return rc;
      if ((rc = check_ref(t.location, t.offset, len, (int64_t)m->len))) return rc;
      if (len < need)
        return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" external data too short");
      b->p = (const uint8_t *)m->base + t.offset;
      b->n = (size_t)need;
      return MMNB_OK;
    }
    if (t.raw.p) {
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
        if (es == 1) b->own[(size_t)i] = (uint8_t)v;
        else if (es == 2) { const uint16_t h = (uint16_t)v; std::memcpy(&b->own[(size_t)(2 * i)], &h, 2); }
        else if (es == 4) { const int32_t w = (int32_t)v; std::memcpy(&b->own[(size_t)(4 * i)], &w, 4); }
        else std::memcpy(&b->own[(size_t)(8 * i)], &v, 8);
      }
      b->p = b->own.data();
      b->n = (size_t)need;
      return MMNB_OK;
    }
    if (cnt == 0) return MMNB_OK;
    return fail(MMNB_ERR_ARG, "Tensor \"" + t.name + "\" has no data");
  }

 private:
  int ext(const std::string &loc, Mapping **out) {
    auto it = maps_.find(loc);
    if (it == maps_.end()) {
      int rc = check_ref(loc, 0, 0, 0);  // path safety before touching disk
      if (rc) return rc;
      std::unique_ptr<Mapping> m(new Mapping());
      if ((rc = map_file(dir_ + "/" + loc, m.get()))) return rc;
      it = maps_.emplace(loc, std::move(m)).first;
    }
    *out = it->second.get();
    return MMNB_OK;
  }
  std::string dir_;
  std::unordered_map<std::string, std::unique_ptr<Mapping>> maps_;
};

int64_t attr_i(const Node &n, const char *name, int64_t dflt, bool *found = nullptr) {
  auto it = n.attrs.find(name);
  const bool ok = it != n.attrs.end() && it->second.has_i;
  if (found) *found = ok;
  return ok ? it->second.i : dflt;
}

// MMNB_DT_F32 / MMNB_DT_F16 for a float initializer, 0 for any other type
// (a uint8 or int32 tensor is not reinterpreted as floats: its byte length
// was checked for its own element size).
int dt_float(int dtype) {
  return dtype == kF16 ? MMNB_DT_F16 : dtype == kF32 ? MMNB_DT_F32 : 0;
}

std::vector<int64_t> to_i64(const Bytes &b) {
  std::vector<int64_t> v((size_t)b.count());
  for (size_t i = 0; i < v.size(); i++)
    v[i] = b.dtype == kI8 ? (int64_t)(int8_t)b.p[i] : (int64_t)b.p[i];
  return v;
}

}  // namespace

extern "C" {

int mmnb_check_external_ref(const char *location, int64_t offset, int64_t length,
                            int64_t file_len) {
  return check_ref(location ? std::string(location) : std::string(), offset, length, file_len);
}

int mmnb_model_free(mmnb_model *m) {
  if (!m) return MMNB_OK;
  for (auto &e : m->entries) (void)mmnb_pack_free(e.pack);
  delete m;
  return MMNB_OK;
}

int mmnb_model_load(mmnb_ctx *ctx, const char *path, mmnb_model **out) {
  MMNB_GUARD_CTX(ctx);
  if (!path || !out) return fail(MMNB_ERR_ARG, "model: null argument");
  *out = nullptr;
  const std::string p(path);
  const size_t slash = p.find_last_of('/');
  const std::string dir = slash == std::string::npos ? "." : p.substr(0, slash);
  Mapping model;
  int rc = map_file(p, &model);
  if (rc) return rc;
  // ModelProto.graph = 7; GraphProto.node = 1, .initializer = 5
  Span graph;
  {
    Reader r(Span{(const uint8_t *)model.base, model.len});
    Field f;
    bool bad = false;
    while (r.next(&f, &bad))
      if (f.no == 7 && f.wt == 2) graph = f.s;
    if (bad) return fail(MMNB_ERR_ARG, "model: malformed protobuf");
  }
  if (!graph.p) return fail(MMNB_ERR_ARG, "model: no graph");
  std::vector<Node> nodes;
  std::unordered_map<std::string, Tensor> inits;
  {
    Reader r(graph);
    Field f;
    bool bad = false;
    while (r.next(&f, &bad)) {
      if (f.wt != 2) continue;
      if (f.no == 1) {
        Node n;
        if (!parse_node(f.s, &n)) return fail(MMNB_ERR_ARG, "model: malformed node");
        nodes.push_back(std::move(n));
      } else if (f.no == 5) {
        Tensor t;
        if (!parse_tensor(f.s, &t)) return fail(MMNB_ERR_ARG, "model: malformed initializer");
        std::string name = t.name;
        inits[name] = std::move(t);
      }
    }
    if (bad) return fail(MMNB_ERR_ARG, "model: malformed graph");
  }
  Loader ld(dir);
  std::unique_ptr<mmnb_model> m(new (std::nothrow) mmnb_model());
  if (!m) return fail(MMNB_ERR_OOM, "out of host memory");
  m->ctx = ctx;
  auto init = [&](const Node &n, size_t i) -> const Tensor * {
    if (i >= n.in.size() || n.in[i].empty()) return nullptr;
    auto it = inits.find(n.in[i]);
    return it == inits.end() ? nullptr : &it->second;
  };
  auto cleanup = [&](int code) {
    mmnb_model_free(m.release());
    return code;
  };
  for (const Node &n : nodes) {
    const std::string label = !n.name.empty() ? n.name : (n.out.empty() ? n.op : n.out[0]);
    mmnb_pack *pack = nullptr;
    if (n.op == "MatMulNBits") {
      const Tensor *tb = init(n, 1), *ts = init(n, 2);
      if (!tb || !ts) continue;
      const bool has_z = n.in.size() > 3 && !n.in[3].empty();
      const bool has_g = n.in.size() > 4 && !n.in[4].empty();
      const bool has_b = n.in.size() > 5 && !n.in[5].empty();
      const Tensor *tz = init(n, 3), *tg = init(n, 4), *tbias = init(n, 5);
      if ((has_z && !tz) || (has_g && !tg) || (has_b && !tbias)) continue;  // dynamic input
      bool fk, fn, fbs;
      mmnb_nbits_desc d{};
      d.k = attr_i(n, "K", 0, &fk);
      d.n = attr_i(n, "N", 0, &fn);
      d.bits = attr_i(n, "bits", 4);
      d.block_size = attr_i(n, "block_size", 0, &fbs);
      if (!fk || !fn || !fbs)
        return cleanup(fail(MMNB_ERR_ARG, "MatMulNBits " + label + ": K, N, block_size required"));
      Bytes bb, bs, bz, bg, bbias;
      if ((rc = ld.bytes(*tb, &bb)) || (rc = ld.bytes(*ts, &bs))) return cleanup(rc);
      if (tb->dtype != kU8) return cleanup(fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: B must be uint8"));
      d.b_q = bb.p;
      d.b_q_len = (int64_t)bb.n;
      d.scales = bs.p;
      d.scales_len = bs.count();
      d.scales_type = dt_float(ts->dtype);
      if (!d.scales_type)
        return cleanup(fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits " + label +
                                                      ": scales must be float or float16"));
      if (tz) {
        if ((rc = ld.bytes(*tz, &bz))) return cleanup(rc);
        d.zero_points = bz.p;
        d.zero_points_len = bz.count();
        d.zero_points_type = tz->dtype == kU8 ? MMNB_DT_U8 : dt_float(tz->dtype);
        if (!d.zero_points_type)
          return cleanup(fail(MMNB_ERR_UNSUPPORTED,
                              "MatMulNBits " + label +
                                  ": zero points must be uint8, float or float16"));
        d.zero_points_layout = tz->dims.size() == 2 ? MMNB_ZP_PER_COLUMN : MMNB_ZP_FLAT;
      }
      std::vector<int32_t> g32;
      if (tg) {
        if ((rc = ld.bytes(*tg, &bg))) return cleanup(rc);
        g32.resize((size_t)bg.count());
        for (size_t i = 0; i < g32.size(); i++) {
          if (tg->dtype == kI64) { int64_t v; std::memcpy(&v, bg.p + 8 * i, 8); g32[i] = (int32_t)v; }
          else if (tg->dtype == kI32) std::memcpy(&g32[i], bg.p + 4 * i, 4);
          else return cleanup(fail(MMNB_ERR_UNSUPPORTED, "MatMulNBits: g_idx must be int32"));
        }
        d.g_idx = g32.data();
        d.g_idx_len = (int64_t)g32.size();
      }
      if (tbias) {
        if ((rc = ld.bytes(*tbias, &bbias))) return cleanup(rc);
        d.bias = bbias.p;
        d.bias_len = bbias.count();
        d.bias_type = dt_float(tbias->dtype);
        if (!d.bias_type)
          return cleanup(fail(MMNB_ERR_UNSUPPORTED,
                              "MatMulNBits " + label + ": bias must be float or float16"));
      }
      if ((rc = mmnb_pack_nbits_ex(ctx, &d, &pack))) return cleanup(rc);
    } else if (n.op == "MatMulInteger" || n.op == "QLinearMatMul") {
      const bool q = n.op == "QLinearMatMul";
      const Tensor *tb = init(n, q ? 3 : 1), *tz = init(n, q ? 5 : 3);
      const size_t zi = q ? 5 : 3;
      if (!tb || (n.in.size() > zi && !n.in[zi].empty() && !tz)) continue;
      Bytes bb, bz;
      if ((rc = ld.bytes(*tb, &bb))) return cleanup(rc);
      if ((tb->dtype != kU8 && tb->dtype != kI8) || tb->dims.size() < 2)
        return cleanup(fail(MMNB_ERR_UNSUPPORTED, n.op + ": B must be uint8/int8, rank >= 2"));
      std::vector<int64_t> z;
      if (tz) {
        if ((rc = ld.bytes(*tz, &bz))) return cleanup(rc);
        if (tz->dtype != kU8 && tz->dtype != kI8)
          return cleanup(fail(MMNB_ERR_UNSUPPORTED, n.op + ": zero point must be uint8/int8"));
        z = to_i64(bz);
      }
      const int64_t kk = tb->dims[tb->dims.size() - 2], nn = tb->dims.back();
      const int64_t batch = kk * nn ? bb.count() / (kk * nn) : 1;
      if ((rc = mmnb_pack_integer(ctx, bb.p, tb->dtype == kI8, batch, kk, nn,
                                  z.empty() ? nullptr : z.data(), (int64_t)z.size(), &pack)))
        return cleanup(rc);
    } else if (n.op == "ConvInteger" || n.op == "QLinearConv") {
      const bool q = n.op == "QLinearConv";
      const Tensor *tw = init(n, q ? 3 : 1), *tz = init(n, q ? 5 : 3);
      const size_t zi = q ? 5 : 3;
      if (!tw || (n.in.size() > zi && !n.in[zi].empty() && !tz)) continue;
      Bytes bw, bz;
      if ((rc = ld.bytes(*tw, &bw))) return cleanup(rc);
      if (tw->dtype != kU8 && tw->dtype != kI8)
        return cleanup(fail(MMNB_ERR_UNSUPPORTED, n.op + ": W must be uint8/int8"));
      std::vector<int64_t> dims = tw->dims;
      if (dims.size() == 3) dims.insert(dims.begin() + 2, 1);  // 1-D as 2-D
      if (dims.size() != 4)
        return cleanup(fail(MMNB_ERR_UNSUPPORTED, n.op + ": 1-D or 2-D convolutions only"));
      std::vector<int64_t> z;
      if (tz) {
        if ((rc = ld.bytes(*tz, &bz))) return cleanup(rc);
        if (tz->dtype != kU8 && tz->dtype != kI8)
          return cleanup(fail(MMNB_ERR_UNSUPPORTED, n.op + ": zero point must be uint8/int8"));
        z = to_i64(bz);
      }
      if ((rc = mmnb_pack_conv(ctx, bw.p, tw->dtype == kI8, dims[0], dims[1], dims[2], dims[3],
                               attr_i(n, "group", 1), z.empty() ? nullptr : z.data(),
                               (int64_t)z.size(), &pack)))
        return cleanup(rc);
    } else {
      continue;
    }
    m->entries.push_back(mmnb_model::Entry{n.op, label, pack});
  }
  *out = m.release();
  return MMNB_OK;
}

int64_t mmnb_model_pack_count(const mmnb_model *m) {
  return m ? (int64_t)m->entries.size() : 0;
}

int mmnb_model_pack_info(const mmnb_model *m, int64_t i, const char **op_type,
                         const char **node_name, const mmnb_pack **pack) {
  if (!m || i < 0 || i >= (int64_t)m->entries.size())
    return fail(MMNB_ERR_ARG, "model: pack index out of range");
  const auto &e = m->entries[(size_t)i];
  if (op_type) *op_type = e.op.c_str();
  if (node_name) *node_name = e.name.c_str();
  if (pack) *pack = e.pack;
  return MMNB_OK;
}

int mmnb_model_find(const mmnb_model *m, const char *node_name, const mmnb_pack **pack) {
  if (!m || !node_name || !pack) return fail(MMNB_ERR_ARG, "model: null argument");
  for (const auto &e : m->entries)
    if (e.name == node_name) {
      *pack = e.pack;
      return MMNB_OK;
    }
  return fail(MMNB_ERR_ARG, std::string("model: no packed node named ") + node_name);
}

}  // extern "C"
