// Manifest directory reader: manifest.json (format kleinhirn-weights-2), its sha256-checked shards
// and the word table (words.bin rows with a murmur3 checksum each, or the legacy keepOnCpu parts).
// Host code only; the device upload lives with the context in runner.hip.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace kh {
namespace mf {

// SHA-256 (FIPS 180-4) of n bytes; the SHA extensions of the CPU when it has them.
void sha256(const void *data, size_t n, uint8_t out[32]);
std::string sha256_hex(const void *data, size_t n);

// Checksum of one words.bin row (src/words-format.ts:18-32): murmur3_32 over the row's
// little-endian u32 words, seeded with salt ^ (row_id + 1) * 0x9e3779b1. n must be a multiple of 4.
uint32_t row_checksum(const uint8_t *row, size_t n, uint32_t row_id, uint32_t salt);

// A read-only mapping of a whole file.
struct MappedFile {
  const uint8_t *p = nullptr;
  size_t n = 0;
  std::string path;
  explicit MappedFile(const std::string &path);
  ~MappedFile();
  MappedFile(const MappedFile &) = delete;
  MappedFile &operator=(const MappedFile &) = delete;
};

struct Tensor {
  std::string name;
  int dtype = 0;  // KH_F32 / KH_F16
  std::vector<int64_t> shape;
  int shard = 0;
  uint64_t offset = 0, bytes = 0;
  bool keep_on_cpu = false;
  int64_t row_start = 0;
};

enum Flags { NO_SHA256 = 1, CHECK_ROWS = 2, NO_WORDS = 4 };

struct Loaded {
  std::string format;
  int version = 0;
  std::vector<Tensor> tensors;                      // every entry of the manifest
  std::vector<std::unique_ptr<MappedFile>> shards;  // checked
  // word table: rows x width values of words_dtype, row i at words_data + i * words_stride
  int words_dtype = -1;
  int64_t words_rows = 0, words_width = 0, words_stride = 0;
  const uint8_t *words_data = nullptr;
  std::unique_ptr<MappedFile> words_file;  // version 3
  std::vector<uint8_t> words_joined;       // legacy: the keepOnCpu parts in row order
  uint64_t file_bytes = 0;
  double read_ms = 0, sha256_ms = 0, rows_ms = 0;
};

// Reads the manifest at `path` and the files it names, with the checks of the reference's loader:
// shard sizes and sha256 (src/weights.ts:150-173), words.bin size, row layout and sha256
// (src/words.ts:98-114), the word table of a legacy manifest (src/weights.ts:67-90). CHECK_ROWS
// also checks every words.bin row against its checksum (src/words-format.ts:34-39). Throws
// std::runtime_error with the reference's messages.
std::unique_ptr<Loaded> load(const std::string &path, int flags);

}  // namespace mf
}  // namespace kh
