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
//
// The file is read by the host-only planner (mmnb_host.cpp, which the CPU
// fuzz harness runs under AddressSanitizer); this file turns its plans into
// device packs.
#include <memory>
#include <string>
#include <vector>

#include "mmnb_host.h"
#include "mmnb_internal.h"

using namespace mmnb;

struct mmnb_model {
  mmnb_ctx *ctx = nullptr;
  struct Entry {
    std::string op, name;
    mmnb_pack *pack = nullptr;
  };
  std::vector<Entry> entries;
};

extern "C" {

int mmnb_check_external_ref(const char *location, int64_t offset, int64_t length,
                            int64_t file_len) {
  return onnx::check_ref(location ? std::string(location) : std::string(), offset, length,
                         file_len);
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
  onnx::MappedFile model;
  int rc = onnx::map_file(p, &model);
  if (rc) return rc;
  onnx::MappedExternalData ext(dir);
  std::vector<onnx::PackPlan> plans;
  if ((rc = onnx::scan_model(model.span(), &ext, &plans))) return rc;
  std::unique_ptr<mmnb_model> m(new (std::nothrow) mmnb_model());
  if (!m) return fail(MMNB_ERR_OOM, "out of host memory");
  m->ctx = ctx;
  for (const onnx::PackPlan &pl : plans) {
    mmnb_pack *pack = nullptr;
    const int64_t *zp = pl.zero_point.empty() ? nullptr : pl.zero_point.data();
    const int64_t zl = (int64_t)pl.zero_point.size();
    if (pl.kind == onnx::kPlanNBits)
      rc = mmnb_pack_nbits_ex(ctx, &pl.nbits, &pack);
    else if (pl.kind == onnx::kPlanInteger)
      rc = mmnb_pack_integer(ctx, pl.w, pl.w_signed, pl.batch, pl.k, pl.n, zp, zl, &pack);
    else
      rc = mmnb_pack_conv(ctx, pl.w, pl.w_signed, pl.co, pl.ci, pl.kh, pl.kw, pl.group, zp, zl,
                          &pack);
    if (rc) {
      mmnb_model_free(m.release());
      return rc;
    }
    m->entries.push_back(mmnb_model::Entry{pl.op, pl.label, pack});
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
