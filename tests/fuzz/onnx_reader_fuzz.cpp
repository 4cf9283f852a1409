// Reader-robustness fuzz harness for libmmnb's host input code
// (onnx_runtime_dart_amd/csrc/mmnb_host.cpp), built for the CPU with
// AddressSanitizer + UBSan by tests/test_onnx_reader_fuzz.py.
//
// The contract (the reference's, tool/fuzz/README.md:1-17): on any input the
// reader parses or rejects with a documented status -- MMNB_ERR_ARG or
// MMNB_ERR_UNSUPPORTED -- never reads outside its input (the sanitizers
// abort on that), never allocates beyond a bound (ASAN_OPTIONS
// max_allocation_size_mb), and never takes long.  For every plan it
// accepts, the harness then reads exactly the bytes the pack entry points
// read (and runs the MatMulNBits host preparation itself), so a plan whose
// spans are shorter than its shapes fails here.
//
// Usage: onnx_reader_fuzz <dir> <iterations> [seed]
//   <dir> holds seed models (*.onnx, which must load as they are), model
//   variants (*.onnx.v: inconsistent shapes, types, attributes and external
//   references, which may be rejected) and the companion files their
//   external data names.  Every seed and variant runs as it is, and every
//   fuzz input is one of them after 1-4 byte mutations; the companion files
//   are handed over as exact-size heap buffers (sometimes truncated).  Exit
//   status 0 when the contract held for every input.
#include <dirent.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "mmnb_host.h"

namespace mmnb {
static std::string g_msg;
int fail(int code, const std::string &msg) {
  g_msg = msg;
  return code;
}
}  // namespace mmnb

using namespace mmnb;
using Bytes = std::vector<uint8_t>;

namespace {

struct Rng {
  uint64_t s;
  uint64_t next() {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
  }
  size_t below(size_t n) { return n ? (size_t)(next() % n) : 0; }
};

// Companion files as heap buffers of exactly their size.
class MemExternal : public onnx::ExternalData {
 public:
  std::map<std::string, Bytes> files;
  // this input's buffers (one per location, like a mapping), freed after it
  std::map<std::string, std::pair<std::unique_ptr<uint8_t[]>, size_t>> live;
  std::map<std::string, size_t> cut;  // truncated length for this input
  int get(const std::string &loc, onnx::Span *out) override {
    auto l = live.find(loc);
    if (l == live.end()) {
      auto it = files.find(loc);
      if (it == files.end()) return fail(MMNB_ERR_ARG, "model: cannot open " + loc);
      size_t n = it->second.size();
      auto c = cut.find(loc);
      if (c != cut.end()) n = c->second;
      std::unique_ptr<uint8_t[]> buf(new uint8_t[n ? n : 1]);
      if (n) std::memcpy(buf.get(), it->second.data(), n);
      l = live.emplace(loc, std::make_pair(std::move(buf), n)).first;
    }
    out->p = l->second.first.get();
    out->n = l->second.second;
    return MMNB_OK;
  }
};

uint64_t g_sink = 0;

void touch(const uint8_t *p, int64_t n) {
  uint64_t h = 0;
  for (int64_t i = 0; i < n; i++) h = h * 31 + p[i];
  g_sink += h;
}

template <typename T>
void touch_vec(const std::vector<T> &v) {
  touch((const uint8_t *)v.data(), (int64_t)(v.size() * sizeof(T)));
}

struct Stats {
  long inputs = 0, ok = 0, arg = 0, unsupported = 0, plans = 0, violations = 0;
  double max_ms = 0;
};

// Runs one input through the planner and the plan consumers.
int run_one(const uint8_t *data, size_t n, MemExternal *ext, Stats *st, const char *what) {
  std::unique_ptr<uint8_t[]> buf(new uint8_t[n ? n : 1]);  // exact size: overreads trap
  if (n) std::memcpy(buf.get(), data, n);
  const auto t0 = std::chrono::steady_clock::now();
  std::vector<onnx::PackPlan> plans;
  int rc = onnx::scan_model(onnx::Span{buf.get(), n}, ext, &plans);
  if (rc == MMNB_OK) {
    for (const onnx::PackPlan &pl : plans) {
      st->plans++;
      if (pl.kind == onnx::kPlanNBits) {
        NbitsHost h;
        const int r2 = nbits_prepare(&pl.nbits, &h);
        if (r2 == MMNB_OK) {
          touch_vec(h.vb);
          touch_vec(h.vs);
          touch_vec(h.vz);
          touch_vec(h.corr);
          touch_vec(h.asrc);
          touch_vec(h.bias);
        } else if (r2 != MMNB_ERR_ARG && r2 != MMNB_ERR_UNSUPPORTED) {
          rc = r2;
        }
      } else if (pl.kind == onnx::kPlanInteger) {
        // mmnb_pack_integer reads batch * k * n bytes of w
        int64_t bk, bkn;
        if (pl.batch >= 1 && pl.n >= 1 && pl.k >= 0 && mul_nonneg(pl.batch, pl.k, &bk) &&
            mul_nonneg(bk, pl.n, &bkn))
          touch(pl.w, bkn);
      } else if (pl.kind == onnx::kPlanConv) {
        // mmnb_pack_conv reads co * ci * kh * kw bytes of w
        int64_t a, b, c;
        if (pl.co >= 1 && pl.ci >= 1 && pl.kh >= 1 && pl.kw >= 1 &&
            mul_nonneg(pl.co, pl.ci, &a) && mul_nonneg(a, pl.kh, &b) &&
            mul_nonneg(b, pl.kw, &c))
          touch(pl.w, c);
      } else {
        std::printf("VIOLATION %s: plan of unknown kind %d\n", what, pl.kind);
        st->violations++;
      }
    }
  }
  const double ms =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  st->inputs++;
  if (ms > st->max_ms) st->max_ms = ms;
  if (rc == MMNB_OK) st->ok++;
  else if (rc == MMNB_ERR_ARG) st->arg++;
  else if (rc == MMNB_ERR_UNSUPPORTED) st->unsupported++;
  else {
    std::printf("VIOLATION %s: undocumented status %d (%s)\n", what, rc, g_msg.c_str());
    st->violations++;
  }
  if (ms > 2000.0) {
    std::printf("VIOLATION %s: took %.0f ms\n", what, ms);
    st->violations++;
  }
  return rc;
}

Bytes read_file(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  return Bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

// Every regular file under dir, by path relative to dir.
void list_files(const std::string &dir, const std::string &rel, std::vector<std::string> *out) {
  DIR *d = opendir((dir + "/" + rel).c_str());
  if (!d) return;
  while (dirent *e = readdir(d)) {
    const std::string name = e->d_name;
    if (name == "." || name == "..") continue;
    const std::string r = rel.empty() ? name : rel + "/" + name;
    if (e->d_type == DT_DIR) list_files(dir, r, out);
    else out->push_back(r);
  }
  closedir(d);
}

void mutate(Bytes *b, Rng *rng) {
  const int kind = (int)rng->below(8);
  const size_t n = b->size();
  switch (kind) {
    case 0:  // flip a bit
      if (n) (*b)[rng->below(n)] ^= (uint8_t)(1u << rng->below(8));
      break;
    case 1:  // set a byte
      if (n) (*b)[rng->below(n)] = (uint8_t)rng->next();
      break;
    case 2: {  // insert random bytes
      const size_t at = rng->below(n + 1), k = 1 + rng->below(8);
      Bytes ins(k);
      for (auto &x : ins) x = (uint8_t)rng->next();
      b->insert(b->begin() + (long)at, ins.begin(), ins.end());
      break;
    }
    case 3:  // delete a range
      if (n) {
        const size_t at = rng->below(n), k = 1 + rng->below(std::min<size_t>(n - at, 64));
        b->erase(b->begin() + (long)at, b->begin() + (long)(at + k));
      }
      break;
    case 4:  // truncate
      b->resize(rng->below(n + 1));
      break;
    case 5:  // a run of continuation bytes (long / overlong varints)
      if (n) {
        const size_t at = rng->below(n), k = 1 + rng->below(12);
        for (size_t i = at; i < std::min(n, at + k); i++) (*b)[i] = 0xFF;
      }
      break;
    case 6: {  // copy a range over another place
      if (n > 2) {
        const size_t src = rng->below(n), dst = rng->below(n);
        const size_t k = 1 + rng->below(std::min<size_t>(n - std::max(src, dst), 32));
        std::memmove(b->data() + dst, b->data() + src, k);
      }
      break;
    }
    default:  // a small or huge value byte (lengths, dims, dtypes)
      if (n) {
        static const uint8_t vals[] = {0x00, 0x01, 0x02, 0x7F, 0x80, 0xFE, 0x10, 0x40};
        (*b)[rng->below(n)] = vals[rng->below(sizeof vals)];
      }
      break;
  }
}

int check_ref_cases() {
  struct C {
    const char *loc;
    int64_t off, len, file;
    bool ok;
  } cases[] = {
      // onnx_runtime_dart_io.dart:44-69 and test/parser_robustness_test.dart
      {"../../etc/passwd", 0, 0, 1 << 20, false},
      {"/etc/passwd", 0, 0, 1 << 20, false},
      {"weights/../../../secret", 0, 0, 1 << 20, false},
      {"C:\\Windows\\x", 0, 0, 1 << 20, false},
      {"", 0, 0, 1 << 20, false},
      {"w.bin", -1, 10, 1000, false},
      {"w.bin", 0, -5, 1000, false},
      {"w.bin", 0, (int64_t)1 << 40, 1000, false},
      {"w.bin", 990, 20, 1000, false},
      {"w.bin", INT64_MAX, 1, 1000, false},
      {"weights.bin", 100, 400, 1000, true},
      {"sub/weights.bin", 0, 1000, 1000, true},
  };
  int bad = 0;
  for (const C &c : cases) {
    const int rc = onnx::check_ref(c.loc, c.off, c.len, c.file);
    if ((rc == MMNB_OK) != c.ok || (rc != MMNB_OK && rc != MMNB_ERR_ARG)) {
      std::printf("VIOLATION check_ref(\"%s\", %lld, %lld, %lld) = %d\n", c.loc,
                  (long long)c.off, (long long)c.len, (long long)c.file, rc);
      bad++;
    }
  }
  return bad;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 3) {
    std::fprintf(stderr, "usage: %s <dir> <iterations> [seed]\n", argv[0]);
    return 2;
  }
  const std::string dir = argv[1];
  const long iters = std::atol(argv[2]);
  Rng rng{argc > 3 ? std::strtoull(argv[3], nullptr, 10) | 1 : 0x9E3779B97F4A7C15ull};
  Stats st;
  st.violations += check_ref_cases();

  MemExternal ext;
  std::vector<std::string> files;
  list_files(dir, "", &files);
  auto ends = [](const std::string &f, const char *suf) {
    const size_t k = std::strlen(suf);
    return f.size() > k && f.compare(f.size() - k, k, suf) == 0;
  };
  std::vector<std::pair<std::string, Bytes>> seeds, bases;
  for (const std::string &f : files) {
    Bytes b = read_file(dir + "/" + f);
    if (ends(f, ".onnx")) seeds.emplace_back(f, b);
    if (ends(f, ".onnx") || ends(f, ".onnx.v")) bases.emplace_back(f, b);
    else ext.files[f] = b;
  }
  // Seeds must load as they are (and exercise every plan kind between them).
  long seed_plans[4] = {0, 0, 0, 0};
  for (const auto &s : seeds) {
    std::vector<onnx::PackPlan> plans;
    const int rc = onnx::scan_model(onnx::Span{s.second.data(), s.second.size()}, &ext, &plans);
    if (rc != MMNB_OK) {
      std::printf("SEED %s rejected: %d %s\n", s.first.c_str(), rc, g_msg.c_str());
      st.violations++;
    }
    for (const auto &p : plans) seed_plans[p.kind & 3]++;
    plans.clear();
    ext.live.clear();
    run_one(s.second.data(), s.second.size(), &ext, &st, s.first.c_str());
    ext.live.clear();
  }
  // Minimized inputs from the reference's reader-robustness tests
  // (test/parser_robustness_test.dart): truncated / huge varints, a
  // truncated length-delimited field, empty input, skipped fields, and a
  // large all-zero blob (no allocation bomb).
  long variants = 0;
  for (const auto &v : bases)
    if (ends(v.first, ".onnx.v")) {
      run_one(v.second.data(), v.second.size(), &ext, &st, v.first.c_str());
      ext.live.clear();
      variants++;
    }
  const std::vector<Bytes> regress = {
      {5}, {0x08}, {0xFF, 0xFF, 0xFF, 0xFF}, {}, {0x12, 0x7F, 0x08}, Bytes(64, 0x0A),
      Bytes(1 << 20, 0)};
  Bytes huge = {0x08};
  huge.insert(huge.end(), 20, 0xFF);
  huge.push_back(0x7F);
  for (const Bytes &r : regress) run_one(r.data(), r.size(), &ext, &st, "regression");
  run_one(huge.data(), huge.size(), &ext, &st, "regression");
  ext.live.clear();

  if (seeds.empty()) {
    std::printf("no seed models in %s\n", dir.c_str());
    return 2;
  }
  for (long i = 0; i < iters; i++) {
    const auto &seed = bases[rng.below(bases.size())];
    Bytes b = seed.second;
    const int muts = 1 + (int)rng.below(4);
    for (int m = 0; m < muts; m++) mutate(&b, &rng);
    ext.cut.clear();
    if (rng.below(10) == 0)
      for (const auto &f : ext.files) ext.cut[f.first] = rng.below(f.second.size() + 1);
    char what[96];
    std::snprintf(what, sizeof what, "input %ld from %s", i, seed.first.c_str());
    run_one(b.data(), b.size(), &ext, &st, what);
    ext.live.clear();
  }
  std::printf(
      "seeds %zu (plans nbits %ld integer %ld conv %ld) variants %ld inputs %ld: ok %ld, "
      "ERR_ARG %ld, ERR_UNSUPPORTED %ld, plans %ld, max %.1f ms, violations %ld (sink %llu)\n",
      seeds.size(), seed_plans[1], seed_plans[2], seed_plans[3], variants, st.inputs, st.ok,
      st.arg, st.unsupported, st.plans, st.max_ms, st.violations,
      (unsigned long long)(g_sink & 1));
  return st.violations ? 1 : 0;
}
