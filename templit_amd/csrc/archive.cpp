// Checkpoint archive (see model_utils/archive.h for the file layout).
// Reference behaviour: src/model_utils/archive.cpp:9-92.
#include "model_utils/archive.h"

#include <cstdint>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <utility>

void Archive::write(const std::string &name, std::span<const std::byte> data) {
  if (!storage.emplace(name, std::vector<std::byte>(data.begin(), data.end())).second)
    throw std::runtime_error("archive already holds an entry named " + name);
}

void Archive::read(const std::string &name, std::span<std::byte> data) const {
  const auto it = storage.find(name);
  if (it == storage.end()) throw std::runtime_error("archive has no entry named " + name);
  if (it->second.size() != data.size())
    throw std::runtime_error("archive entry " + name + " has " +
                             std::to_string(it->second.size()) + " bytes, not " +
                             std::to_string(data.size()));
  if (!data.empty()) std::memcpy(data.data(), it->second.data(), data.size());
}

std::vector<std::string> Archive::names() const {
  std::vector<std::string> out;
  out.reserve(storage.size());
  for (const auto &entry : storage) out.push_back(entry.first);
  return out;
}

ArchiveView Archive::scope(const std::string &name) { return ArchiveView(this, name); }

namespace {
void put_u32(std::ostream &out, size_t v) {
  if (v > std::numeric_limits<uint32_t>::max())
    throw std::runtime_error("archive entry exceeds 4 GiB");
  const uint32_t x = static_cast<uint32_t>(v);
  out.write(reinterpret_cast<const char *>(&x), sizeof(x));
}
} // namespace

void Archive::commit(std::ostream &out) const {
  for (const auto &[name, blob] : storage) {
    put_u32(out, name.size());
    out.write(name.data(), std::streamsize(name.size()));
    put_u32(out, blob.size());
    out.write(reinterpret_cast<const char *>(blob.data()), std::streamsize(blob.size()));
  }
}

void Archive::restore(std::istream &in) {
  for (;;) {
    uint32_t name_len = 0, blob_len = 0;
    if (!in.read(reinterpret_cast<char *>(&name_len), sizeof(name_len))) return;
    std::string name(name_len, '\0');
    if (!in.read(name.data(), name_len)) return;
    if (!in.read(reinterpret_cast<char *>(&blob_len), sizeof(blob_len))) return;
    std::vector<std::byte> blob(blob_len);
    if (!in.read(reinterpret_cast<char *>(blob.data()), blob_len)) return;
    storage[std::move(name)] = std::move(blob); // a later entry replaces an earlier one
  }
}

ArchiveView::ArchiveView(Archive *archive, std::string_view prefix)
    : archive_(archive), prefix_(prefix) {}

void ArchiveView::write(const std::string &name, std::span<const std::byte> data) {
  archive_->write(prefix_ + "/" + name, data);
}

void ArchiveView::read(const std::string &name, std::span<std::byte> data) const {
  archive_->read(prefix_ + "/" + name, data);
}

ArchiveView ArchiveView::scope(const std::string &name) const {
  return ArchiveView(archive_, prefix_ + "/" + name);
}
