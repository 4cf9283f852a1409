// Host-only parts of libmmnb that read untrusted input: the ONNX wire reader
// that turns a model file into pack plans, and the host preparation of
// MatMulNBits weights (mmnb_pack_nbits_ex).  No HIP here, so the same source
// builds with g++ for the CPU under AddressSanitizer / UBSan and the fuzz
// harness (tests/fuzz/onnx_reader_fuzz.cpp) drives it directly.
//
// Contract on any input (the reference's reader-robustness contract,
// tool/fuzz/README.md:1-17, test/parser_robustness_test.dart): parse, or
// reject with a documented status (MMNB_ERR_ARG for malformed or
// out-of-range data, MMNB_ERR_UNSUPPORTED for valid ONNX outside what the
// kernels take), never read outside the bytes it was given, and allocate in
// proportion to the input only.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mmnb.h"

namespace mmnb {

// Sets the thread's last-error message and returns code (libmmnb's one
// error path; mmnb_last_error() reads the message).
int fail(int code, const std::string &msg);

// a * b for a, b >= 0 into *out; false when the product exceeds INT64_MAX.
inline bool mul_nonneg(int64_t a, int64_t b, int64_t *out) {
  if (a < 0 || b < 0) return false;
  if (a != 0 && b > INT64_MAX / a) return false;
  *out = a * b;
  return true;
}

// ---- MatMulNBits host preparation.  The kernels run on a 4-bit "virtual"
// weight of kv rows with zero point 8 or packed uint4 zero points; every
// extension of the operator (bits 8, g_idx, bias, float zero points, fp16
// scales, per-column zero-point layout) is turned into that weight plus an
// optional A gather (asrc) and a correction pass (corr, bias) here.
struct NbitsHost {
  int64_t k = 0, n = 0, block = 0, n_blocks = 0;  // the operator's K, N
  int64_t kv = 0;                 // rows of the virtual weight
  std::vector<uint8_t> vb;        // [n][ceil(kv / block)][block / 2] nibbles
  std::vector<float> vs;          // [n][ceil(kv / block)] scales
  std::vector<uint8_t> vz;        // flat packed uint4 zero points, or empty
  int zfill = 0x88;               // zero-point filler byte when vz is empty
  std::vector<double> corr;       // [n_blocks][n], or empty
  std::vector<int32_t> asrc;      // [kv] column of A per virtual row (-1: 0)
  std::vector<float> bias;        // [n], or empty
};

// Validates d against its own lengths and builds the virtual weight.
int nbits_prepare(const mmnb_nbits_desc *d, NbitsHost *out);

// IEEE-754 binary16 -> binary32 (exact).
float half_to_float(uint16_t h);

namespace onnx {

struct Span {
  const uint8_t *p = nullptr;
  size_t n = 0;
};

// The reference's guard on an external-data reference
// (checkExternalRef, onnx_runtime_dart_io.dart:44-69): a relative location
// inside the model's directory, and [offset, offset + length) inside the
// companion file.
int check_ref(const std::string &loc, int64_t off, int64_t len, int64_t file_len);

// Source of external-data files, by location relative to the model.
class ExternalData {
 public:
  virtual ~ExternalData() {}
  // The whole file named by loc (already checked by check_ref).
  virtual int get(const std::string &loc, Span *out) = 0;
};

// A read-only memory mapping of a file.
struct MappedFile {
  void *base = nullptr;
  size_t len = 0;
  MappedFile() = default;
  MappedFile(const MappedFile &) = delete;
  MappedFile &operator=(const MappedFile &) = delete;
  ~MappedFile();
  Span span() const { return Span{(const uint8_t *)base, len}; }
};
int map_file(const std::string &path, MappedFile *m);

// External data memory-mapped from files under a directory.
class MappedExternalData : public ExternalData {
 public:
  explicit MappedExternalData(const std::string &dir) : dir_(dir) {}
  int get(const std::string &loc, Span *out) override;

 private:
  std::string dir_;
  std::unordered_map<std::string, std::unique_ptr<MappedFile>> maps_;
};

// One initializer's bytes: a span of the model or of a companion file, or
// decoded from an inline typed list into `own`.
struct WeightBytes {
  const uint8_t *p = nullptr;
  size_t n = 0;                 // = count * element size
  int dtype = 0;                // TensorProto.DataType
  std::vector<int64_t> dims;
  int64_t count = 0;
  std::vector<uint8_t> own;
};

enum PlanKind { kPlanNBits = 1, kPlanInteger = 2, kPlanConv = 3 };

// One weight pack to build: the node's op type and label, and the
// arguments of mmnb_pack_nbits_ex / mmnb_pack_integer / mmnb_pack_conv.
// Pointers refer to the model or companion mappings or to `keep`.
struct PackPlan {
  int kind = 0;
  std::string op, label;
  mmnb_nbits_desc nbits{};        // kPlanNBits
  std::vector<int32_t> g_idx;     // kPlanNBits: g_idx as int32
  const uint8_t *w = nullptr;     // kPlanInteger / kPlanConv
  bool w_signed = false;
  int64_t batch = 0, k = 0, n = 0;               // kPlanInteger: w is [batch, k, n]
  int64_t co = 0, ci = 0, kh = 0, kw = 0, group = 1;  // kPlanConv: w is [co, ci, kh, kw]
  std::vector<int64_t> zero_point;
  std::vector<WeightBytes> keep;
};

// Walks the graph of the ModelProto in `model` and plans a pack for every
// MatMulNBits, MatMulInteger, QLinearMatMul, ConvInteger and QLinearConv
// whose weight inputs are initializers (nodes with dynamic weights are
// skipped).  The plans point into `model` and into ext's spans.
int scan_model(Span model, ExternalData *ext, std::vector<PackPlan> *plans);

}  // namespace onnx
}  // namespace mmnb
