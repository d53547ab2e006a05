// Host-only driver for the checkpoint reader under AddressSanitizer / UBSan
// (tests/test_checkpoint_asan.py builds it with csrc/checkpoint.hip compiled for the
// host only).  For every file argument it opens the checkpoint, reads every tensor's
// bytes, queries the EXL3 linear geometry of every name prefix and closes it.  With
// --mutate SEED N FILE it also writes N copies of FILE with 1..8 random bytes of its
// header (or its length) changed and runs each through the same sequence.  Only parsing
// is exercised: the GPU entry points it references are stubs.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <random>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "../include/crucible_exl3.h"

extern "C" {
// The reader's upload path is never called here; these satisfy the link only.
int cx_exl3_repack(const int16_t*, int32_t, int32_t, int32_t, uint32_t*, cx_stream_t) { return CX_E_UNSUPPORTED; }
hipError_t hipMemcpyAsync(void*, const void*, size_t, hipMemcpyKind, hipStream_t) { return hipErrorNotSupported; }
hipError_t hipStreamSynchronize(hipStream_t) { return hipErrorNotSupported; }
}

static uint64_t g_sum = 0;

static int Exercise(const char* path) {
  cx_checkpoint* ck = nullptr;
  const int rc = cx_checkpoint_open(path, &ck);
  if (rc != 0) {
    g_sum += std::strlen(cx_last_error());
    return 0;
  }
  const int n = cx_checkpoint_count(ck);
  for (int i = 0; i < n; ++i) {
    const char* name = cx_checkpoint_name(ck, i);
    int32_t dt = 0, rank = 0;
    int64_t shape[CX_MAX_RANK];
    const void* data = nullptr;
    uint64_t bytes = 0;
    if (cx_checkpoint_tensor(ck, name, &dt, &rank, shape, &data, &bytes) == 0 && data) {
      const unsigned char* p = static_cast<const unsigned char*>(data);
      for (uint64_t b = 0; b < bytes; ++b) g_sum += p[b];
    }
    std::string prefix(name);
    const size_t dot = prefix.find_last_of('.');
    if (dot != std::string::npos) prefix.resize(dot);
    int32_t I = 0, O = 0, k2 = 0, cb = 0;
    (void)cx_exl3_linear_info(ck, prefix.c_str(), &I, &O, &k2, &cb);
    g_sum += (uint64_t)(I + O + k2 + cb);
  }
  cx_checkpoint_close(ck);
  return 1;
}

int main(int argc, char** argv) {
  int opened = 0, files = 0;
  for (int a = 1; a < argc; ++a) {
    if (std::strcmp(argv[a], "--mutate") == 0 && a + 3 < argc) {
      const unsigned seed = (unsigned)std::strtoul(argv[a + 1], nullptr, 10);
      const int count = std::atoi(argv[a + 2]);
      const char* src = argv[a + 3];
      a += 3;
      std::ifstream in(src, std::ios::binary);
      std::vector<char> orig((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
      if (orig.size() < 8) return 2;
      uint64_t hlen = 0;
      std::memcpy(&hlen, orig.data(), 8);
      const size_t span = (size_t)std::min<uint64_t>(orig.size(), hlen + 8);
      std::mt19937 rng(seed);
      const std::string tmp = std::string(src) + ".mut";
      for (int k = 0; k < count; ++k) {
        std::vector<char> m = orig;
        const int edits = 1 + (int)(rng() % 8);
        for (int e = 0; e < edits; ++e) {
          const uint32_t kind = rng() % 8;
          const size_t at = rng() % span;
          if (kind == 0) m[at] = "{}[]\",:0123456789eE.-\\ "[rng() % 24];
          else if (kind == 1) m.resize(at);  // truncated file
          else if (kind == 2 && at < 8) m[at] = (char)(rng() & 0xff);  // header length
          else if (at < m.size()) m[at] = (char)(rng() & 0xff);
          if (m.size() < 8) break;
        }
        std::ofstream(tmp, std::ios::binary | std::ios::trunc).write(m.data(), (std::streamsize)m.size());
        opened += Exercise(tmp.c_str());
        ++files;
      }
      std::remove(tmp.c_str());
      continue;
    }
    opened += Exercise(argv[a]);
    ++files;
  }
  std::printf("files %d opened %d checksum %llu\n", files, opened, (unsigned long long)g_sum);
  return 0;
}
