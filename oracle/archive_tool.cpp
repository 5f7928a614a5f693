// archive_tool -- the reference's checkpoint Archive (src/model_utils/
// archive.cpp, compiled where it lies by oracle/Makefile) writing and
// reading files, to pin the file layout of templit_amd's own Archive.
// TEST INFRASTRUCTURE ONLY.
//   archive_tool write FILE   the fixed test archive, through the reference API
//   archive_tool dump FILE    one line per entry: name, size, FNV-1a 64 of the bytes
// The same two modes exist in tests/cpp/test_archive.cpp over templit_amd's
// Archive; the outputs must be identical.
#include "archive_tool_content.h"
#include "model_utils/archive.h"

#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>

int main(int argc, char **argv) {
  if (argc != 3) return 2;
  try {
    if (std::strcmp(argv[1], "write") == 0) {
      Archive a;
      archive_test_content::write_all(a);
      std::ofstream out(argv[2], std::ios::binary);
      a.commit(out);
      return out.good() ? 0 : 1;
    }
    if (std::strcmp(argv[1], "dump") == 0) {
      std::ifstream in(argv[2], std::ios::binary);
      Archive a;
      a.restore(in);
      archive_test_content::dump(a, archive_test_content::names_in_file(argv[2]));
      return 0;
    }
  } catch (const std::exception &e) {
    std::fprintf(stderr, "archive_tool: %s\n", e.what());
    return 1;
  }
  return 2;
}
