// Checkpoint archive: named byte blobs with "/"-scoped names, written to and
// read from a stream. Same interface and file layout as the reference's
// Archive (include/model_utils/archive.h:15-43, src/model_utils/
// archive.cpp:9-92), so a checkpoint moves between the reference's CPU or
// Metal builds and this one in either direction:
//   file = { u32 name_length, name bytes, u32 blob_length, blob bytes }*
// in native (little-endian) byte order, entries in any order; a truncated
// trailing entry ends the read. Names are unique: writing one twice throws.
// Here the entries are kept sorted by name, so a file's bytes depend only on
// its contents.
#pragma once

#include "model_utils/archive_concepts.h"

#include <cstddef>
#include <istream>
#include <map>
#include <ostream>
#include <span>
#include <string>
#include <string_view>
#include <vector>

class ArchiveView;

class Archive {
  std::map<std::string, std::vector<std::byte>> storage;

public:
  // Throws std::runtime_error if `name` exists.
  void write(const std::string &name, std::span<const std::byte> data);
  // Throws std::runtime_error if `name` is missing or its size differs.
  void read(const std::string &name, std::span<std::byte> data) const;
  bool contains(const std::string &name) const { return storage.count(name) != 0; }
  // Entry names in sorted order (not in the reference interface).
  std::vector<std::string> names() const;

  ArchiveView scope(const std::string &name);

  void commit(std::ostream &out) const;
  void restore(std::istream &in);
};

// Names relative to a prefix: scope("a").write("b") writes "a/b".
class ArchiveView {
  Archive *archive_;
  std::string prefix_;
  ArchiveView(Archive *archive, std::string_view prefix);
  friend class Archive;

public:
  void write(const std::string &name, std::span<const std::byte> data);
  void read(const std::string &name, std::span<std::byte> data) const;
  ArchiveView scope(const std::string &name) const;
};

static_assert(ArchiveType<Archive>);
static_assert(ArchiveType<ArchiveView>);
