// Manifest directory reader (see manifest.h). Host code, built with the system C++ compiler.
#include "manifest.h"

#include <fcntl.h>
#include <immintrin.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <thread>

#include "../../include/kh_hip.h"
#include "json.h"

namespace kh {
namespace mf {

namespace {

// ---- SHA-256 --------------------------------------------------------------------------------

// Round constants and initial state from their definition (FIPS 180-4 4.2.2, 5.3.3): the first 32
// bits of the fractional parts of the cube roots of the first 64 primes and of the square roots of
// the first 8, computed with exact integer roots.
struct ShaConstants {
  uint32_t k[64], h0[8];
  ShaConstants() {
    int primes[64], n = 0;
    for (int c = 2; n < 64; c++) {
      bool prime = true;
      for (int d = 2; d * d <= c; d++) prime = prime && c % d != 0;
      if (prime) primes[n++] = c;
    }
    typedef unsigned __int128 u128;
    auto iroot = [](u128 v, int e) {  // floor(v^(1/e)) for e = 2, 3
      uint64_t lo = 0, hi = (uint64_t)1 << 40;
      while (lo < hi) {
        const uint64_t mid = (lo + hi + 1) / 2;
        u128 p = (u128)mid * mid;
        if (e == 3) p *= mid;
        if (p <= v) lo = mid;
        else hi = mid - 1;
      }
      return lo;
    };
    for (int i = 0; i < 64; i++) k[i] = (uint32_t)iroot((u128)primes[i] << 96, 3);
    for (int i = 0; i < 8; i++) h0[i] = (uint32_t)iroot((u128)primes[i] << 64, 2);
  }
};
const ShaConstants kSha;

inline uint32_t rotr(uint32_t x, int r) { return (x >> r) | (x << (32 - r)); }
inline uint32_t rotl(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }
inline uint32_t be32(const uint8_t *p) {
  return (uint32_t)p[0] << 24 | (uint32_t)p[1] << 16 | (uint32_t)p[2] << 8 | (uint32_t)p[3];
}

void blocks_portable(uint32_t st[8], const uint8_t *p, size_t nblk) {
  uint32_t w[64];
  for (; nblk; nblk--, p += 64) {
    for (int t = 0; t < 16; t++) w[t] = be32(p + 4 * t);
    for (int t = 16; t < 64; t++) {
      const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
      const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
      w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = st[0], b = st[1], c = st[2], d = st[3], e = st[4], f = st[5], g = st[6], h = st[7];
    for (int t = 0; t < 64; t++) {
      const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + kSha.k[t] + w[t];
      const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    st[0] += a; st[1] += b; st[2] += c; st[3] += d;
    st[4] += e; st[5] += f; st[6] += g; st[7] += h;
  }
}

// The same compression with the x86 SHA extensions: sha256rnds2 runs two rounds on the state
// held as (A, B, E, F) and (C, D, G, H); msg1 / msg2 extend the schedule four words at a time.
__attribute__((target("sha,sse4.1"))) void blocks_shani(uint32_t st[8], const uint8_t *p, size_t nblk) {
  const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bULL, 0x0405060700010203ULL);
  __m128i dcba = _mm_loadu_si128((const __m128i *)&st[0]);
  __m128i hgfe = _mm_loadu_si128((const __m128i *)&st[4]);
  const __m128i cdab = _mm_shuffle_epi32(dcba, 0xB1);
  const __m128i efgh = _mm_shuffle_epi32(hgfe, 0x1B);
  __m128i abef = _mm_alignr_epi8(cdab, efgh, 8);
  __m128i cdgh = _mm_blend_epi16(efgh, cdab, 0xF0);
  for (; nblk; nblk--, p += 64) {
    const __m128i abef0 = abef, cdgh0 = cdgh;
    __m128i w[4];
    for (int i = 0; i < 4; i++) w[i] = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i *)(p + 16 * i)), bswap);
    for (int i = 0; i < 16; i++) {
      if (i >= 4) {
        // w[i % 4] becomes words 4 i .. 4 i + 3 from words 4 i - 16 .. 4 i - 1
        __m128i x = _mm_sha256msg1_epu32(w[i & 3], w[(i + 1) & 3]);
        x = _mm_add_epi32(x, _mm_alignr_epi8(w[(i + 3) & 3], w[(i + 2) & 3], 4));
        w[i & 3] = _mm_sha256msg2_epu32(x, w[(i + 3) & 3]);
      }
      // two rounds leave (A, B, E, F) in the first operand's place and the old one becomes (C, D, G, H)
      __m128i m = _mm_add_epi32(w[i & 3], _mm_loadu_si128((const __m128i *)&kSha.k[4 * i]));
      cdgh = _mm_sha256rnds2_epu32(cdgh, abef, m);
      m = _mm_shuffle_epi32(m, 0x0E);
      abef = _mm_sha256rnds2_epu32(abef, cdgh, m);
    }
    abef = _mm_add_epi32(abef, abef0);
    cdgh = _mm_add_epi32(cdgh, cdgh0);
  }
  const __m128i feba = _mm_shuffle_epi32(abef, 0x1B);
  const __m128i dchg = _mm_shuffle_epi32(cdgh, 0xB1);
  dcba = _mm_blend_epi16(feba, dchg, 0xF0);
  hgfe = _mm_alignr_epi8(dchg, feba, 8);
  _mm_storeu_si128((__m128i *)&st[0], dcba);
  _mm_storeu_si128((__m128i *)&st[4], hgfe);
}

bool use_shani() {
  static const bool yes = __builtin_cpu_supports("sha") && __builtin_cpu_supports("sse4.1") &&
                          !getenv("KH_SHA256_PORTABLE");
  return yes;
}

double ms_since(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t).count();
}

[[noreturn]] void fail(const std::string &m) { throw std::runtime_error(m); }

}  // namespace

void sha256(const void *data, size_t n, uint8_t out[32]) {
  uint32_t st[8];
  memcpy(st, kSha.h0, sizeof st);
  const uint8_t *p = (const uint8_t *)data;
  const size_t full = n / 64;
  auto blocks = use_shani() ? blocks_shani : blocks_portable;
  if (full) blocks(st, p, full);
  // the tail, 0x80, zeros and the bit length (big-endian) in one or two blocks
  uint8_t tail[128] = {};
  const size_t rest = n - full * 64;
  if (rest) memcpy(tail, p + full * 64, rest);
  tail[rest] = 0x80;
  const size_t tb = rest + 9 <= 64 ? 64 : 128;
  const uint64_t bits = (uint64_t)n * 8;
  for (int i = 0; i < 8; i++) tail[tb - 1 - i] = (uint8_t)(bits >> (8 * i));
  blocks(st, tail, tb / 64);
  for (int i = 0; i < 8; i++) {
    out[4 * i] = (uint8_t)(st[i] >> 24);
    out[4 * i + 1] = (uint8_t)(st[i] >> 16);
    out[4 * i + 2] = (uint8_t)(st[i] >> 8);
    out[4 * i + 3] = (uint8_t)st[i];
  }
}

std::string sha256_hex(const void *data, size_t n) {
  uint8_t d[32];
  sha256(data, n, d);
  static const char *hx = "0123456789abcdef";
  std::string s(64, '0');
  for (int i = 0; i < 32; i++) {
    s[2 * i] = hx[d[i] >> 4];
    s[2 * i + 1] = hx[d[i] & 15];
  }
  return s;
}

uint32_t row_checksum(const uint8_t *row, size_t n, uint32_t row_id, uint32_t salt) {
  uint32_t h = salt ^ (uint32_t)((row_id + 1u) * 0x9e3779b1u);
  for (size_t i = 0; i + 4 <= n; i += 4) {
    uint32_t k;
    memcpy(&k, row + i, 4);  // little-endian host
    k *= 0xcc9e2d51u;
    k = rotl(k, 15);
    k *= 0x1b873593u;
    h ^= k;
    h = rotl(h, 13);
    h = h * 5u + 0xe6546b64u;
  }
  h ^= (uint32_t)n;
  h ^= h >> 16;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  h *= 0xc2b2ae35u;
  h ^= h >> 16;
  return h;
}

MappedFile::MappedFile(const std::string &file) : path(file) {
  const int fd = open(file.c_str(), O_RDONLY);
  if (fd < 0) fail("cannot open " + file + ": " + strerror(errno));
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    close(fd);
    fail("cannot stat " + file);
  }
  n = (size_t)sb.st_size;
  if (n > 0) {
    void *m = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      close(fd);
      fail("cannot map " + file + ": " + strerror(errno));
    }
    madvise(m, n, MADV_SEQUENTIAL);
    p = (const uint8_t *)m;
  }
  close(fd);
}

MappedFile::~MappedFile() {
  if (p) munmap((void *)p, n);
}

namespace {

int dtype_of(const std::string &name, const std::string &d) {
  if (d == "f16") return KH_F16;
  if (d == "f32") return KH_F32;
  fail("tensor " + name + ": dtype " + d + " (f16 or f32)");
}

// sha256 of each file on its own thread; returns the summed hashing time
double check_sha(const std::vector<std::pair<const MappedFile *, std::string>> &files) {
  std::vector<std::string> got(files.size());
  std::vector<double> ms(files.size());
  std::vector<std::thread> th;
  for (size_t i = 0; i < files.size(); i++)
    th.emplace_back([&, i] {
      const auto t = std::chrono::steady_clock::now();
      got[i] = sha256_hex(files[i].first->p, files[i].first->n);
      ms[i] = ms_since(t);
    });
  for (auto &t : th) t.join();
  double sum = 0;
  for (size_t i = 0; i < files.size(); i++) {
    sum += ms[i];
    if (got[i] != files[i].second) {
      const std::string &p = files[i].first->path;
      fail("sha256 mismatch on " + p.substr(p.find_last_of('/') + 1));
    }
  }
  return sum;
}

}  // namespace

std::unique_ptr<Loaded> load(const std::string &path, int flags) {
  auto L = std::make_unique<Loaded>();
  const auto t0 = std::chrono::steady_clock::now();
  const std::string base = path.find('/') == std::string::npos ? "" : path.substr(0, path.find_last_of('/') + 1);
  Json m;
  {
    MappedFile f(path);
    try {
      m = JsonReader((const char *)f.p, f.n).parse();
    } catch (const std::runtime_error &e) {
      fail(path + ": " + e.what());
    }
  }
  try {
    L->format = m.has("format") ? m.at("format").str() : "";
    L->version = m.has("version") ? (int)m.at("version").integer() : 0;
    for (const Json &t : m.at("tensors").arr()) {
      Tensor x;
      x.name = t.at("name").str();
      x.dtype = dtype_of(x.name, t.at("dtype").str());
      for (const Json &d : t.at("shape").arr()) x.shape.push_back(d.integer());
      x.shard = (int)t.at("shard").integer();
      x.offset = (uint64_t)t.at("offset").integer();
      x.bytes = (uint64_t)t.at("byteLength").integer();
      x.keep_on_cpu = t.has("keepOnCpu") && t.at("keepOnCpu").kind == Json::Bool && t.at("keepOnCpu").b;
      x.row_start = t.has("rowStart") ? t.at("rowStart").integer() : 0;
      int64_t count = 1;
      for (int64_t d : x.shape) count *= d;
      if ((uint64_t)count * (x.dtype == KH_F16 ? 2 : 4) != x.bytes)
        fail("tensor " + x.name + ": " + std::to_string(x.bytes) + " bytes for shape of " + std::to_string(count) +
             " elements");
      L->tensors.push_back(std::move(x));
    }
    std::vector<std::pair<const MappedFile *, std::string>> hashed;
    const std::vector<Json> &shards = m.at("shards").arr();
    for (const Json &s : shards) {
      L->shards.emplace_back(new MappedFile(base + s.at("file").str()));
      const MappedFile &f = *L->shards.back();
      if (s.has("bytes") && (uint64_t)s.at("bytes").integer() != f.n)
        fail(s.at("file").str() + " is " + std::to_string(f.n) + " bytes, manifest says " +
             std::to_string(s.at("bytes").integer()));
      hashed.push_back({&f, s.at("sha256").str()});
      L->file_bytes += f.n;
    }
    for (const Tensor &t : L->tensors) {
      if (t.shard < 0 || t.shard >= (int)L->shards.size())
        fail("tensor " + t.name + ": shard " + std::to_string(t.shard) + " of " + std::to_string(L->shards.size()));
      if (t.offset + t.bytes > L->shards[t.shard]->n)
        fail("tensor " + t.name + " runs past the end of " + m.at("shards").arr()[t.shard].at("file").str());
    }
    // word table
    const bool want_words = !(flags & NO_WORDS);
    if (m.has("words") && m.at("words").kind == Json::Obj) {
      const Json &w = m.at("words");
      const std::string file = w.at("file").str();
      const std::string dt = w.at("dtype").str();
      const int es = dt == "f16" ? 2 : 4;
      if (dt != "f16" && dt != "f32") fail("words: dtype " + dt);
      const int64_t rows = w.at("rows").integer(), width = w.at("width").integer();
      const int64_t row_bytes = w.at("rowBytes").integer();
      if (row_bytes != width * es + 4)
        fail("words: rowBytes " + std::to_string(row_bytes) + " is not " + std::to_string(width) + " " + dt +
             " values and a checksum");
      if (want_words) {
        L->words_file.reset(new MappedFile(base + file));
        const MappedFile &f = *L->words_file;
        const int64_t declared = w.at("bytes").integer();
        if ((int64_t)f.n != declared)
          fail("words.bin is " + std::to_string(f.n) + " bytes, manifest says " + std::to_string(declared));
        if ((int64_t)f.n != rows * row_bytes)
          fail("words.bin is " + std::to_string(f.n) + " bytes, " + std::to_string(rows) + " rows of " +
               std::to_string(row_bytes) + " need " + std::to_string(rows * row_bytes));
        hashed.push_back({&f, w.at("sha256").str()});
        L->file_bytes += f.n;
        L->words_dtype = dt == "f16" ? KH_F16 : KH_F32;
        L->words_rows = rows;
        L->words_width = width;
        L->words_stride = row_bytes;
        L->words_data = f.p;
        if (flags & CHECK_ROWS) {
          const uint32_t salt = (uint32_t)w.at("salt").integer();
          const auto t = std::chrono::steady_clock::now();
          for (int64_t i = 0; i < rows; i++) {
            const uint8_t *r = f.p + i * row_bytes;
            uint32_t stored;
            memcpy(&stored, r + row_bytes - 4, 4);
            if (row_checksum(r, (size_t)row_bytes - 4, (uint32_t)i, salt) != stored)
              fail("words.bin row " + std::to_string(i) + " fails its checksum");
          }
          L->rows_ms = ms_since(t);
        }
      }
    } else if (want_words) {
      // legacy: the keepOnCpu parts of the shards joined in row order; their shape holds the width
      std::vector<const Tensor *> parts;
      for (const Tensor &t : L->tensors)
        if (t.keep_on_cpu) parts.push_back(&t);
      if (parts.empty()) fail("manifest has neither words.bin nor a keepOnCpu word table");
      std::stable_sort(parts.begin(), parts.end(), [](const Tensor *a, const Tensor *b) { return a->row_start < b->row_start; });
      uint64_t total = 0;
      for (const Tensor *t : parts) {
        if (t->name != "embeddings.word.weight") fail("only the word table stays on the CPU");
        if (t->shape.size() != 2 || t->shape[1] != parts[0]->shape[1] || t->dtype != parts[0]->dtype)
          fail("word table parts differ in width or dtype");
        total += t->bytes;
      }
      L->words_joined.resize(total);
      uint64_t at = 0;
      for (const Tensor *t : parts) {
        memcpy(L->words_joined.data() + at, L->shards[t->shard]->p + t->offset, t->bytes);
        at += t->bytes;
      }
      const int es = parts[0]->dtype == KH_F16 ? 2 : 4;
      L->words_dtype = parts[0]->dtype;
      L->words_width = parts[0]->shape[1];
      L->words_rows = (int64_t)(total / (uint64_t)(es * L->words_width));
      L->words_stride = es * L->words_width;
      L->words_data = L->words_joined.data();
    }
    L->read_ms = ms_since(t0);
    if (!(flags & NO_SHA256)) L->sha256_ms = check_sha(hashed);
  } catch (const std::runtime_error &e) {
    const std::string what = e.what();
    // the JSON reader names plan documents; say which document it was
    if (what.rfind("plan JSON", 0) == 0) fail(path + ": " + what.substr(5));
    throw;
  }
  return L;
}

}  // namespace mf
}  // namespace kh
