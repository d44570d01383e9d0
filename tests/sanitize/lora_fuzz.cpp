// lora_fuzz.cpp -- the 'LORA' v1 reader (glacier.tune_amd/csrc/lora_file.cpp)
// under AddressSanitizer and UndefinedBehaviorSanitizer, fed truncated and
// corrupted files (tests/test_sanitizers.py builds and runs it).
//
//   lora_fuzz <work dir> <random cases>
//
// A valid file (long names with two-byte length prefixes, an empty-name
// record, several shapes) is written with lora::save and read back exactly.
// Then every prefix of it, every single-byte change at the header and record
// boundaries, a set of hand-made hostile records (huge or negative
// dimensions, an over-long name length, a name length varint that never
// ends) and <random cases> random multi-byte corruptions are each read with
// the same loop a caller uses: open, then next/read until the records end,
// retrying a too-small name buffer once, reading each payload into an
// exactly-sized heap block (or skipping it when it is implausibly large).
// Every call must return OK, INVALID_ARGUMENT or DATA; anything else, or a
// sanitizer report, fails the run.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../../glacier.tune_amd/csrc/lora_file.hpp"

namespace lora = glacier::lora;

namespace {

int g_fail = 0;

void expect_code(int rc, const char* what) {
  if (rc != GLACIER_ATTN_OK && rc != GLACIER_ATTN_ERR_INVALID_ARGUMENT && rc != GLACIER_LORA_ERR_DATA) {
    std::fprintf(stderr, "unexpected status %d from %s\n", rc, what);
    g_fail = 1;
  }
}

std::vector<unsigned char> slurp(const std::string& path) {
  std::vector<unsigned char> out;
  FILE* f = std::fopen(path.c_str(), "rb");
  if (f == nullptr) return out;
  unsigned char buf[4096];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) out.insert(out.end(), buf, buf + n);
  std::fclose(f);
  return out;
}

void spit(const std::string& path, const std::vector<unsigned char>& bytes) {
  FILE* f = std::fopen(path.c_str(), "wb");
  if (f == nullptr) {
    std::perror("fopen");
    std::exit(2);
  }
  if (!bytes.empty()) std::fwrite(bytes.data(), 1, bytes.size(), f);
  std::fclose(f);
}

// Reads the whole file the way a caller does; returns the number of records
// read in full.
int read_all(const std::string& path, std::vector<std::vector<float>>* payloads = nullptr) {
  std::string err;
  glacier_lora_header h{};
  glacier_lora_reader* r = nullptr;
  int rc = lora::open(path.c_str(), &h, &r, err);
  expect_code(rc, "open");
  if (rc != GLACIER_ATTN_OK) return 0;
  int done = 0;
  for (int i = 0; i < h.tensor_count && i < 64; ++i) {
    char small[8];
    int32_t d0 = 0, d1 = 0;
    rc = lora::next(r, small, sizeof(small), &d0, &d1, err);
    expect_code(rc, "next (small buffer)");
    if (rc == GLACIER_ATTN_ERR_INVALID_ARGUMENT) {
      std::vector<char> name(1 << 16);
      rc = lora::next(r, name.data(), static_cast<int32_t>(name.size()), &d0, &d1, err);
      expect_code(rc, "next");
    }
    if (rc != GLACIER_ATTN_OK) break;
    const long long n = static_cast<long long>(d0) * d1;
    if (d0 <= 0 || d1 <= 0) {
      std::fprintf(stderr, "next accepted dims %d x %d\n", d0, d1);
      g_fail = 1;
      break;
    }
    if (n > (1LL << 22)) {
      rc = lora::read(r, nullptr, 0, err);  // skip
      expect_code(rc, "read (skip)");
    } else {
      std::vector<float>* dst = nullptr;
      std::vector<float> local;
      if (payloads != nullptr) {
        payloads->emplace_back();
        dst = &payloads->back();
      } else {
        dst = &local;
      }
      dst->assign(static_cast<size_t>(n), 0.0f);
      float* heap = static_cast<float*>(std::malloc(static_cast<size_t>(n) * sizeof(float)));
      rc = lora::read(r, heap, (i & 1) && payloads == nullptr ? 1 : 0, err);
      expect_code(rc, "read");
      if (rc == GLACIER_ATTN_OK) std::memcpy(dst->data(), heap, static_cast<size_t>(n) * sizeof(float));
      std::free(heap);
    }
    if (rc != GLACIER_ATTN_OK) break;
    ++done;
  }
  lora::close(r);
  return done;
}

void put_u32(std::vector<unsigned char>& b, uint32_t v) {
  for (int i = 0; i < 4; ++i) b.push_back(static_cast<unsigned char>(v >> (8 * i)));
}

void put_f32(std::vector<unsigned char>& b, float f) {
  uint32_t v;
  std::memcpy(&v, &f, 4);
  put_u32(b, v);
}

std::vector<unsigned char> header(int32_t count) {
  std::vector<unsigned char> b;
  put_u32(b, GLACIER_LORA_MAGIC);
  put_u32(b, GLACIER_LORA_VERSION);
  put_u32(b, 1);   // layer_count
  put_u32(b, 4);   // rank
  put_f32(b, 8.0f);
  put_u32(b, static_cast<uint32_t>(count));
  return b;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: lora_fuzz <work dir> <random cases>\n");
    return 2;
  }
  const std::string dir = argv[1];
  const int cases = std::atoi(argv[2]);
  const std::string good = dir + "/good.bin", bad = dir + "/case.bin";

  // a valid file
  const std::string long_name(200, 'n');  // two-byte 7-bit length prefix
  std::vector<std::string> names = {"blk.0.attn_q.lora_a.weight", long_name, "",
                                    "blk.3.ffn_down.lora_b.weight"};
  std::vector<int32_t> d0 = {8, 3, 1, 5}, d1 = {4, 7, 1, 2};
  std::vector<std::vector<float>> data;
  for (size_t i = 0; i < names.size(); ++i) {
    data.emplace_back(static_cast<size_t>(d0[i]) * d1[i]);
    for (size_t j = 0; j < data.back().size(); ++j) data.back()[j] = static_cast<float>(i * 100 + j) * 0.25f;
  }
  std::vector<const char*> cnames;
  std::vector<const float*> cdata;
  for (size_t i = 0; i < names.size(); ++i) {
    cnames.push_back(names[i].c_str());
    cdata.push_back(data[i].data());
  }
  std::string err;
  int rc = lora::save(good.c_str(), 1, 4, 8.0f, static_cast<int32_t>(names.size()), cnames.data(),
                      d0.data(), d1.data(), cdata.data(), err);
  if (rc != GLACIER_ATTN_OK) {
    std::fprintf(stderr, "save failed: %s\n", err.c_str());
    return 1;
  }
  std::vector<std::vector<float>> back;
  if (read_all(good, &back) != static_cast<int>(names.size()) || back != data) {
    std::fprintf(stderr, "the valid file did not read back exactly\n");
    return 1;
  }
  const std::vector<unsigned char> bytes = slurp(good);

  // every prefix
  for (size_t n = 0; n < bytes.size(); ++n) {
    spit(bad, std::vector<unsigned char>(bytes.begin(), bytes.begin() + static_cast<long>(n)));
    if (read_all(bad) == static_cast<int>(names.size())) {
      std::fprintf(stderr, "a file cut to %zu of %zu bytes read in full\n", n, bytes.size());
      g_fail = 1;
    }
  }
  // every byte of the header and of the first record's length and dims,
  // set to each of a few values
  const unsigned char vals[] = {0x00, 0x01, 0x7f, 0x80, 0xff};
  for (size_t i = 0; i < 24 + 1 + names[0].size() + 8 && i < bytes.size(); ++i)
    for (unsigned char v : vals) {
      std::vector<unsigned char> b = bytes;
      b[i] = v;
      spit(bad, b);
      read_all(bad);
    }
  // hostile records
  {
    std::vector<std::vector<unsigned char>> hostile;
    auto record = [](std::vector<unsigned char> b, const std::vector<unsigned char>& name_len,
                     int32_t a0, int32_t a1, size_t payload_floats) {
      b.insert(b.end(), name_len.begin(), name_len.end());
      b.push_back('x');
      put_u32(b, static_cast<uint32_t>(a0));
      put_u32(b, static_cast<uint32_t>(a1));
      for (size_t i = 0; i < payload_floats; ++i) put_f32(b, 1.0f);
      return b;
    };
    hostile.push_back(record(header(1), {1}, 0x7fffffff, 0x7fffffff, 4));     // overflowing size
    hostile.push_back(record(header(1), {1}, -3, 4, 4));                       // negative dim
    hostile.push_back(record(header(1), {1}, 0, 4, 0));                        // zero dim
    hostile.push_back(record(header(1), {0xff, 0xff, 0xff, 0xff, 0x07}, 1, 1, 1));  // 2^31-1 name
    hostile.push_back(record(header(1), {0x80, 0x80, 0x80, 0x80, 0x80, 0x01}, 1, 1, 1));  // runaway varint
    hostile.push_back(record(header(3), {1}, 2, 2, 4));                        // count > records
    hostile.push_back(header(-1));                                             // negative count
    hostile.push_back(record(header(1), {1}, 1 << 20, 1 << 12, 16));           // 16 GB claimed, 64 B given
    for (const auto& h : hostile) {
      spit(bad, h);
      read_all(bad);
    }
  }
  // random corruptions
  std::mt19937 rng(12345);
  for (int c = 0; c < cases; ++c) {
    std::vector<unsigned char> b = bytes;
    const int edits = 1 + static_cast<int>(rng() % 4);
    for (int e = 0; e < edits; ++e) b[rng() % b.size()] = static_cast<unsigned char>(rng());
    if (rng() % 4 == 0) b.resize(rng() % b.size());
    spit(bad, b);
    read_all(bad);
  }
  // a missing file and a directory without adapter_model.bin
  read_all(dir + "/missing.bin");
  read_all(dir);
  if (g_fail) return 1;
  std::printf("LORA_FUZZ_OK\n");
  return 0;
}
