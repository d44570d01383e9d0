// lora_file.cpp -- the 'LORA' v1 adapter binary: writer (GgufLoraModel.
// SaveAdapter, src/Glacier.Tune/Model/GgufLoraModel.cs:636-650, with
// TuneBlockSerialization.WriteTensor, ITuneBlock.cs:43-50) and reader with the
// checks of GgufLoraModel.LoadAdapter (:697-796).  Host code; little-endian.
#include "lora_file.hpp"

#include <sys/stat.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

struct glacier_lora_reader {
  FILE* f = nullptr;
  long size = 0;           // bytes in the file
  int32_t left = 0;        // records not yet started
  bool pending = false;    // a record's payload is next in the file
  bool failed = false;     // a malformed or truncated record was met: every later call fails
  int32_t dim0 = 0, dim1 = 0;
};

namespace glacier {
namespace lora {
namespace {

constexpr int kOk = GLACIER_ATTN_OK;
constexpr int kInvalid = GLACIER_ATTN_ERR_INVALID_ARGUMENT;
constexpr int kData = GLACIER_LORA_ERR_DATA;

int bad(std::string& err, int code, const std::string& msg) {
  err = msg;
  return code;
}

bool is_dir(const char* p) {
  struct stat st;
  return stat(p, &st) == 0 && S_ISDIR(st.st_mode);
}

bool is_file(const char* p) {
  struct stat st;
  return stat(p, &st) == 0 && S_ISREG(st.st_mode);
}

bool put(FILE* f, const void* p, size_t n) { return std::fwrite(p, 1, n, f) == n; }

// A .NET BinaryWriter string: the UTF-8 byte count as a 7-bit varint, then
// the bytes.
bool put_string(FILE* f, const char* s) {
  uint32_t n = static_cast<uint32_t>(std::strlen(s));
  unsigned char buf[5];
  int k = 0;
  while (n >= 0x80) {
    buf[k++] = static_cast<unsigned char>(n | 0x80);
    n >>= 7;
  }
  buf[k++] = static_cast<unsigned char>(n);
  return put(f, buf, k) && put(f, s, std::strlen(s));
}

long remaining(const glacier_lora_reader* r) { return r->size - std::ftell(r->f); }

}  // namespace

int save(const char* path, int32_t layer_count, int32_t rank, float alpha, int32_t n_tensors,
         const char* const* names, const int32_t* dim0, const int32_t* dim1,
         const float* const* data, std::string& err) {
  if (path == nullptr) return bad(err, kInvalid, "path is NULL");
  if (n_tensors < 0) return bad(err, kInvalid, "n_tensors must be >= 0");
  if (n_tensors > 0 && (names == nullptr || dim0 == nullptr || dim1 == nullptr || data == nullptr))
    return bad(err, kInvalid, "names, dim0, dim1 and data are required");
  for (int32_t i = 0; i < n_tensors; ++i) {
    if (names[i] == nullptr || data[i] == nullptr)
      return bad(err, kInvalid, "tensor " + std::to_string(i) + ": name or data is NULL");
    if (dim0[i] <= 0 || dim1[i] <= 0)
      return bad(err, kInvalid, "tensor " + std::to_string(i) + ": dimensions must be positive");
  }
  const std::string tmp = std::string(path) + ".tmp";
  FILE* f = std::fopen(tmp.c_str(), "wb");
  if (f == nullptr) return bad(err, kData, "cannot create " + tmp);
  const uint32_t magic = GLACIER_LORA_MAGIC, version = GLACIER_LORA_VERSION;
  bool ok = put(f, &magic, 4) && put(f, &version, 4) && put(f, &layer_count, 4) &&
            put(f, &rank, 4) && put(f, &alpha, 4) && put(f, &n_tensors, 4);
  for (int32_t i = 0; ok && i < n_tensors; ++i) {
    ok = put_string(f, names[i]) && put(f, &dim0[i], 4) && put(f, &dim1[i], 4) &&
         put(f, data[i], sizeof(float) * static_cast<size_t>(dim0[i]) * dim1[i]);
  }
  ok = (std::fclose(f) == 0) && ok;
  if (!ok || std::rename(tmp.c_str(), path) != 0) {
    std::remove(tmp.c_str());
    return bad(err, kData, std::string("writing ") + path + " failed");
  }
  return kOk;
}

int open(const char* path, glacier_lora_header* header, glacier_lora_reader** reader,
         std::string& err) {
  if (path == nullptr || header == nullptr || reader == nullptr)
    return bad(err, kInvalid, "path, header and reader are required");
  *reader = nullptr;
  std::string file = path;
  if (!is_file(path)) {
    const std::string in_dir = std::string(path) + "/adapter_model.bin";
    if (!(is_dir(path) && is_file(in_dir.c_str())))
      return bad(err, kData, std::string("LoRA adapter file not found: ") + path);
    file = in_dir;
  }
  FILE* f = std::fopen(file.c_str(), "rb");
  if (f == nullptr) return bad(err, kData, "cannot open " + file);
  auto r = new glacier_lora_reader;
  r->f = f;
  std::fseek(f, 0, SEEK_END);
  r->size = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  uint32_t magic = 0, version = 0;
  int32_t layers = 0, rank = 0, count = 0;
  float alpha = 0.0f;
  const bool got = std::fread(&magic, 4, 1, f) == 1 && std::fread(&version, 4, 1, f) == 1 &&
                   std::fread(&layers, 4, 1, f) == 1 && std::fread(&rank, 4, 1, f) == 1 &&
                   std::fread(&alpha, 4, 1, f) == 1 && std::fread(&count, 4, 1, f) == 1;
  int code = kOk;
  char hex[16];
  std::snprintf(hex, sizeof(hex), "0x%08X", magic);
  if (!got)
    code = bad(err, kData, "truncated LoRA header");
  else if (magic != GLACIER_LORA_MAGIC)
    code = bad(err, kData, std::string("invalid LoRA magic header: ") + hex + " (expected 0x41524F4C 'LORA')");
  else if (version != GLACIER_LORA_VERSION)
    code = bad(err, kData, "unsupported LoRA adapter version: " + std::to_string(version));
  else if (count < 0)
    code = bad(err, kData, "invalid negative LoRA tensor count: " + std::to_string(count));
  else if (rank > 0 && (!std::isfinite(alpha) || alpha <= 0.0f))
    code = bad(err, kData, "invalid LoRA adapter alpha value: " + std::to_string(alpha));
  if (code != kOk) {
    close(r);
    return code;
  }
  *header = glacier_lora_header{version, layers, rank, alpha, count};
  r->left = count;
  *reader = r;
  return kOk;
}

// The record header at the current position.  A name buffer that is too
// small leaves the reader at the record's start, so a retry with a larger
// buffer reads the same record; a malformed or truncated record marks the
// reader failed (every later next/read returns GLACIER_LORA_ERR_DATA).
int next(glacier_lora_reader* r, char* name, int32_t name_cap, int32_t* dim0, int32_t* dim1,
         std::string& err) {
  if (r == nullptr || name == nullptr || dim0 == nullptr || dim1 == nullptr)
    return bad(err, kInvalid, "reader, name, dim0 and dim1 are required");
  if (r->failed) return bad(err, kData, "the LoRA file was found malformed by an earlier call");
  if (r->pending) return bad(err, kInvalid, "the previous record has not been read or skipped");
  if (r->left <= 0) return bad(err, kInvalid, "no more records");
  const long start = std::ftell(r->f);
  auto corrupt = [&](const std::string& msg) {
    r->failed = true;
    return bad(err, kData, msg);
  };
  // the name: a 7-bit varint byte count, then UTF-8
  uint32_t len = 0;
  int shift = 0;
  for (;;) {
    const int c = std::fgetc(r->f);
    if (c == EOF) return corrupt("truncated LoRA record name");
    len |= static_cast<uint32_t>(c & 0x7F) << shift;
    if ((c & 0x80) == 0) break;
    shift += 7;
    if (shift > 28) return corrupt("malformed LoRA record name length");
  }
  if (static_cast<long>(len) > remaining(r)) return corrupt("truncated LoRA record name");
  if (name_cap <= 0 || static_cast<uint64_t>(len) + 1 > static_cast<uint64_t>(name_cap)) {
    if (std::fseek(r->f, start, SEEK_SET) != 0) return corrupt("seek failed");
    return bad(err, kInvalid, "name buffer too small: the record name needs " +
                                  std::to_string(len + 1) + " bytes");
  }
  if (std::fread(name, 1, len, r->f) != len) return corrupt("truncated LoRA record name");
  name[len] = '\0';
  int32_t d0 = 0, d1 = 0;
  if (std::fread(&d0, 4, 1, r->f) != 1 || std::fread(&d1, 4, 1, r->f) != 1)
    return corrupt(std::string("truncated LoRA record header for '") + name + "'");
  if (d0 <= 0 || d1 <= 0)
    return corrupt("invalid LoRA tensor dimensions [" + std::to_string(d0) + ", " +
                   std::to_string(d1) + "] for '" + name + "'");
  // (2^31 - 1)^2 * 4 bytes still fits 64 unsigned bits
  const uint64_t bytes = static_cast<uint64_t>(d0) * static_cast<uint64_t>(d1) * sizeof(float);
  if (bytes > static_cast<uint64_t>(remaining(r)))
    return corrupt(std::string("truncated LoRA binary payload for '") + name + "': expected " +
                   std::to_string(bytes) + " bytes, only " + std::to_string(remaining(r)) +
                   " remaining");
  r->pending = true;
  r->dim0 = d0;
  r->dim1 = d1;
  r->left -= 1;
  *dim0 = d0;
  *dim1 = d1;
  return kOk;
}

int read(glacier_lora_reader* r, float* dst, int32_t transpose, std::string& err) {
  if (r == nullptr) return bad(err, kInvalid, "reader is NULL");
  if (r->failed) return bad(err, kData, "the LoRA file was found malformed by an earlier call");
  if (!r->pending) return bad(err, kInvalid, "no record is pending: call glacier_lora_next first");
  const size_t n = static_cast<size_t>(r->dim0) * r->dim1;
  r->pending = false;
  auto corrupt = [&](const char* msg) {
    r->failed = true;
    return bad(err, kData, msg);
  };
  if (dst == nullptr) {
    if (std::fseek(r->f, static_cast<long>(n * sizeof(float)), SEEK_CUR) != 0)
      return corrupt("seek failed");
    return kOk;
  }
  if (!transpose) {
    if (std::fread(dst, sizeof(float), n, r->f) != n) return corrupt("truncated LoRA payload");
    return kOk;
  }
  std::vector<float> tmp(n);
  if (std::fread(tmp.data(), sizeof(float), n, r->f) != n) return corrupt("truncated LoRA payload");
  for (int32_t i = 0; i < r->dim0; ++i)
    for (int32_t j = 0; j < r->dim1; ++j)
      dst[static_cast<size_t>(j) * r->dim0 + i] = tmp[static_cast<size_t>(i) * r->dim1 + j];
  return kOk;
}

void close(glacier_lora_reader* r) {
  if (r == nullptr) return;
  if (r->f != nullptr) std::fclose(r->f);
  delete r;
}

}  // namespace lora
}  // namespace glacier
