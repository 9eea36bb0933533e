// GGUF (v2/v3) reader, host side: maps the file read-only and indexes its metadata and tensor table, so tensors can
// be handed to qmatmul_prepare_weight straight from the mapping. Follows the published GGUF layout (magic "GGUF",
// version, tensor count, key-value count, key-values, tensor infos, data aligned to general.alignment); the role of
// the reference's src/gguf.h:85-305, with POSIX mmap in place of its Win32 mapping. A split model
// (name-00001-of-0000N.gguf, "split.count" > 1) opened from its first part maps the other parts too and adds their
// tensors (src/gguf.h:170-187); a later part opened on its own has only its own tensors.
#pragma once
#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace qm {

// GGUF metadata value types
enum GgufVType : uint32_t {
  GV_U8 = 0, GV_I8 = 1, GV_U16 = 2, GV_I16 = 3, GV_U32 = 4, GV_I32 = 5, GV_F32 = 6, GV_BOOL = 7, GV_STR = 8,
  GV_ARR = 9, GV_U64 = 10, GV_I64 = 11, GV_F64 = 12
};

struct GgufValue {
  uint32_t type = 0, elem_type = 0;  // elem_type for arrays
  int64_t i = 0;                     // integer and bool scalars
  double f = 0.0;                    // float scalars
  std::string s;                     // string scalar
  uint64_t count = 0;                // array length
};

struct GgufTensorInfo {
  std::string name;
  uint32_t type = 0, n_dims = 0;
  uint64_t dims[8] = {};             // dims[0] is the contiguous (innermost) dimension
  uint64_t offset = 0, nbytes = 0;
  const uint8_t* data = nullptr;
};

// elements and bytes per block of a GGML type; false for a type this table does not know
bool ggml_type_block(uint32_t type, int& blk, int& bytes);

class Gguf {
 public:
  static std::unique_ptr<Gguf> open(const std::string& path, std::string& err);
  ~Gguf();
  uint32_t version = 0;
  std::vector<std::string> keys;
  std::unordered_map<std::string, GgufValue> kv;
  std::vector<GgufTensorInfo> tensors;
  std::unordered_map<std::string, size_t> index;

 private:
  Gguf() = default;
  bool parse(std::string& err);
  bool open_parts(const std::string& path, std::string& err);
  std::vector<std::unique_ptr<Gguf>> parts_;  // the other parts of a split model (their mappings stay open)
  const uint8_t* base_ = nullptr;
  uint64_t size_ = 0;
  int fd_ = -1;
};

}  // namespace qm
