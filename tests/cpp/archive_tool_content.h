// The fixed content of the archive-format tests, written through any
// archive type with the reference's interface (write / read / scope), and
// a dump of an archive file: one line per entry, sorted by name, with the
// entry's size and the FNV-1a 64 hash of its bytes. Shared by
// oracle/archive_tool.cpp (the reference's Archive) and
// tests/cpp/test_archive.cpp (templit_amd's). TEST INFRASTRUCTURE ONLY.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <span>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace archive_test_content {

inline std::vector<std::byte> pattern(size_t n, uint32_t seed) {
  std::vector<std::byte> v(n);
  uint32_t x = seed * 2654435761u + 1u;
  for (auto &b : v) {
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    b = std::byte(x & 0xff);
  }
  return v;
}

// A checkpoint-shaped archive: scoped parameter and optimiser entries of
// several sizes, an empty entry, a long name, and a record of whether a
// second write of one name was refused.
template <typename Archive> void write_all(Archive &a) {
  auto params = a.scope("parameters");
  const uint32_t shapes[3][2] = {{4, 8}, {1, 8}, {37, 3}};
  for (uint32_t i = 0; i < 3; ++i) {
    auto t = params.scope(std::to_string(i));
    t.write("size", std::as_bytes(std::span<const uint32_t>(shapes[i], 2)));
    t.write("data", pattern(4 * shapes[i][0] * shapes[i][1], i + 1));
  }
  auto opt = a.scope("optimisers").scope("0");
  opt.scope("momentum1").write("data", pattern(128, 10));
  opt.scope("momentum2").write("data", pattern(128, 11));
  const uint32_t step = 7;
  opt.write("step", std::as_bytes(std::span<const uint32_t>(&step, 1)));
  a.write("empty", std::span<const std::byte>());
  a.write(std::string(300, 'n'), pattern(10000, 12));
  uint8_t refused = 0;
  try {
    a.write("empty", pattern(3, 13));
  } catch (const std::runtime_error &) {
    refused = 1;
  }
  a.write("duplicate_refused", std::as_bytes(std::span<const uint8_t>(&refused, 1)));
}

// (name, size) of every complete entry in the file, in file order.
inline std::vector<std::pair<std::string, uint32_t>> names_in_file(const char *path) {
  std::ifstream in(path, std::ios::binary | std::ios::ate);
  const std::streamoff file_size = in.tellg();
  in.seekg(0);
  std::vector<std::pair<std::string, uint32_t>> out;
  for (;;) {
    uint32_t n = 0, size = 0;
    if (!in.read(reinterpret_cast<char *>(&n), 4)) break;
    std::string name(n, '\0');
    if (!in.read(name.data(), n) || !in.read(reinterpret_cast<char *>(&size), 4)) break;
    if (std::streamoff(in.tellg()) + size > file_size) break; // truncated blob
    in.seekg(size, std::ios::cur);
    out.emplace_back(std::move(name), size);
  }
  return out;
}

template <typename Archive>
void dump(const Archive &a, std::vector<std::pair<std::string, uint32_t>> entries) {
  std::sort(entries.begin(), entries.end());
  for (const auto &[name, size] : entries) {
    std::vector<std::byte> blob(size);
    a.read(name, std::span<std::byte>(blob));
    uint64_t h = 1469598103934665603ull;
    for (std::byte b : blob) h = (h ^ uint64_t(b)) * 1099511628211ull;
    std::printf("%s\t%u\t%016llx\n", name.c_str(), size, static_cast<unsigned long long>(h));
  }
}

} // namespace archive_test_content
