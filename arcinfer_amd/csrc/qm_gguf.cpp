// GGUF reader (host C++, POSIX mmap). Every read is bounds-checked against the mapping before it happens, so a
// truncated or hostile file yields an error message, never an out-of-range read.
#include "qm_gguf.h"

#include <cstdio>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace qm {

bool ggml_type_block(uint32_t type, int& blk, int& bytes) {
  // (GGML type ids and block geometry, fixed by the file format)
  struct E { uint32_t t; int blk, bytes; };
  static const E table[] = {
      {0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
      {8, 32, 34},    {9, 32, 36},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
      {14, 256, 210}, {15, 256, 292}, {16, 256, 66},  {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
      {20, 32, 18},   {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {24, 1, 1},     {25, 1, 2},
      {26, 1, 4},     {27, 1, 8},     {28, 1, 8},     {29, 256, 56},  {30, 1, 2},     {39, 32, 17},   {42, 64, 18},
  };
  for (const E& e : table)
    if (e.t == type) {
      blk = e.blk;
      bytes = e.bytes;
      return true;
    }
  return false;
}

namespace {

struct Reader {
  const uint8_t* p;
  uint64_t size, pos = 0;
  bool ok = true;
  bool need(uint64_t n) {
    if (!ok || n > size - pos) ok = false;  // (pos never passes size: the difference cannot wrap)
    return ok;
  }
  template <typename T> T rd() {
    T v{};
    if (need(sizeof(T))) {
      memcpy(&v, p + pos, sizeof(T));
      pos += sizeof(T);
    }
    return v;
  }
  std::string str() {
    const uint64_t n = rd<uint64_t>();
    if (!need(n)) return {};
    std::string s((const char*)p + pos, (size_t)n);
    pos += n;
    return s;
  }
  bool skip(uint64_t n) {
    if (!need(n)) return false;
    pos += n;
    return true;
  }
};

int scalar_bytes(uint32_t t) {
  switch (t) {
    case GV_U8: case GV_I8: case GV_BOOL: return 1;
    case GV_U16: case GV_I16: return 2;
    case GV_U32: case GV_I32: case GV_F32: return 4;
    case GV_U64: case GV_I64: case GV_F64: return 8;
    default: return 0;
  }
}

void read_scalar(Reader& r, uint32_t t, GgufValue& v) {
  switch (t) {
    case GV_U8: v.i = r.rd<uint8_t>(); break;
    case GV_I8: v.i = r.rd<int8_t>(); break;
    case GV_U16: v.i = r.rd<uint16_t>(); break;
    case GV_I16: v.i = r.rd<int16_t>(); break;
    case GV_U32: v.i = r.rd<uint32_t>(); break;
    case GV_I32: v.i = r.rd<int32_t>(); break;
    case GV_U64: v.i = (int64_t)r.rd<uint64_t>(); break;
    case GV_I64: v.i = r.rd<int64_t>(); break;
    case GV_BOOL: v.i = r.rd<uint8_t>() != 0; break;
    case GV_F32: v.f = r.rd<float>(); v.i = (int64_t)v.f; break;
    case GV_F64: v.f = r.rd<double>(); v.i = (int64_t)v.f; break;
    default: r.ok = false;
  }
  if (t != GV_F32 && t != GV_F64) v.f = (double)v.i;
}

}  // namespace

std::unique_ptr<Gguf> Gguf::open(const std::string& path, std::string& err) {
  std::unique_ptr<Gguf> g(new Gguf());
  g->fd_ = ::open(path.c_str(), O_RDONLY);
  if (g->fd_ < 0) {
    err = "cannot open " + path;
    return nullptr;
  }
  struct stat st;
  if (fstat(g->fd_, &st) != 0 || st.st_size <= 0) {
    err = "cannot stat " + path + " (or it is empty)";
    return nullptr;
  }
  g->size_ = (uint64_t)st.st_size;
  void* m = mmap(nullptr, (size_t)g->size_, PROT_READ, MAP_SHARED, g->fd_, 0);
  if (m == MAP_FAILED) {
    err = "cannot map " + path;
    return nullptr;
  }
  g->base_ = (const uint8_t*)m;
  if (!g->parse(err)) return nullptr;
  if (!g->open_parts(path, err)) return nullptr;
  return g;
}

// name-00001-of-0000N.gguf with split.count = N > 1: parts 2..N (same name, part number in the same 5 digits), their
// tensors appended unless a name is already indexed (src/gguf.h:170-187). A part that is missing or malformed fails
// the open.
bool Gguf::open_parts(const std::string& path, std::string& err) {
  const auto it = kv.find("split.count");
  if (it == kv.end() || it->second.type == GV_STR || it->second.type == GV_ARR || it->second.type == GV_F32 ||
      it->second.type == GV_F64)
    return true;
  const int64_t n = it->second.i;
  if (n <= 1) return true;
  const size_t at = path.rfind("-00001-of-");
  if (at == std::string::npos) return true;  // (a later part opened on its own: only its own tensors)
  if (n > 99999) {
    err = "split.count " + std::to_string(n) + " out of range";
    return false;
  }
  for (int64_t k = 2; k <= n; ++k) {
    char num[8];
    snprintf(num, sizeof num, "%05d", (int)k);
    std::string pp = path;
    pp.replace(at + 1, 5, num);
    std::string perr;
    std::unique_ptr<Gguf> part = open(pp, perr);
    if (!part) {
      err = "split part " + std::to_string(k) + " of " + std::to_string(n) + ": " + perr;
      return false;
    }
    for (const GgufTensorInfo& t : part->tensors) {
      if (index.count(t.name)) continue;
      index[t.name] = tensors.size();
      tensors.push_back(t);
    }
    parts_.push_back(std::move(part));
  }
  return true;
}

Gguf::~Gguf() {
  if (base_) munmap((void*)base_, (size_t)size_);
  if (fd_ >= 0) ::close(fd_);
}

bool Gguf::parse(std::string& err) {
  Reader r{base_, size_};
  if (r.rd<uint32_t>() != 0x46554747u || !r.ok) {
    err = "not a GGUF file (magic)";
    return false;
  }
  version = r.rd<uint32_t>();
  if (version < 2 || version > 3) {
    err = "unsupported GGUF version " + std::to_string(version);
    return false;
  }
  const uint64_t nt = r.rd<uint64_t>(), nkv = r.rd<uint64_t>();
  // (a key-value takes at least 13 bytes, a tensor info at least 24: counts the file cannot hold are refused before
  //  anything is allocated for them)
  if (!r.ok || nkv > (size_ - r.pos) / 13 || nt > (size_ - r.pos) / 24) {
    err = "bad tensor or key count";
    return false;
  }
  for (uint64_t i = 0; i < nkv && r.ok; ++i) {
    std::string key = r.str();
    GgufValue v;
    v.type = r.rd<uint32_t>();
    if (v.type == GV_STR) {
      v.s = r.str();
    } else if (v.type == GV_ARR) {
      v.elem_type = r.rd<uint32_t>();
      v.count = r.rd<uint64_t>();
      if (v.elem_type == GV_STR) {
        for (uint64_t k = 0; k < v.count && r.ok; ++k) r.skip(r.rd<uint64_t>());
      } else {
        const int eb = scalar_bytes(v.elem_type);
        if (eb == 0 || v.count > (size_ - r.pos) / (uint64_t)eb) r.ok = false;
        else r.skip(v.count * (uint64_t)eb);
      }
    } else {
      read_scalar(r, v.type, v);
    }
    if (!r.ok) break;
    if (!kv.count(key)) keys.push_back(key);
    kv[key] = v;
  }
  if (!r.ok) {
    err = "truncated or malformed metadata";
    return false;
  }
  tensors.resize(nt);
  for (uint64_t i = 0; i < nt && r.ok; ++i) {
    GgufTensorInfo& t = tensors[i];
    t.name = r.str();
    t.n_dims = r.rd<uint32_t>();
    if (t.n_dims > 8) {
      err = "bad dimension count for " + t.name;
      return false;
    }
    for (uint32_t d = 0; d < t.n_dims; ++d) t.dims[d] = r.rd<uint64_t>();
    t.type = r.rd<uint32_t>();
    t.offset = r.rd<uint64_t>();
    index[t.name] = i;
  }
  if (!r.ok) {
    err = "truncated tensor table";
    return false;
  }
  int64_t align = 32;
  auto it = kv.find("general.alignment");
  if (it != kv.end()) align = it->second.i;
  if (align <= 0 || align > (1 << 20) || (align & (align - 1))) {
    err = "bad general.alignment";
    return false;
  }
  const uint64_t data_start = (r.pos + (uint64_t)align - 1) / (uint64_t)align * (uint64_t)align;
  if (data_start > size_) {
    err = "truncated before the tensor data";
    return false;
  }
  for (GgufTensorInfo& t : tensors) {
    int blk = 0, bytes = 0;
    if (!ggml_type_block(t.type, blk, bytes)) {
      err = "unknown tensor type " + std::to_string(t.type) + " for " + t.name;
      return false;
    }
    uint64_t ne = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
      if (t.dims[d] && ne > UINT64_MAX / t.dims[d]) {
        err = "bad shape for " + t.name;
        return false;
      }
      ne *= t.dims[d];
    }
    if (ne % (uint64_t)blk || ne / (uint64_t)blk > UINT64_MAX / (uint64_t)bytes) {
      err = "shape of " + t.name + " is not whole blocks of its type";
      return false;
    }
    t.nbytes = ne / (uint64_t)blk * (uint64_t)bytes;
    if (t.offset > size_ - data_start || t.nbytes > size_ - data_start - t.offset) {
      err = "tensor data out of the file for " + t.name;
      return false;
    }
    t.data = base_ + data_start + t.offset;
  }
  return true;
}

}  // namespace qm
