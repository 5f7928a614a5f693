// test_archive -- templit_amd's checkpoint Archive writing and reading
// files, for comparison with the reference's (oracle/archive_tool.cpp).
// Host only, no GPU.
//   test_archive write FILE | dump FILE   (see archive_tool_content.h)
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
    std::fprintf(stderr, "test_archive: %s\n", e.what());
    return 1;
  }
  return 2;
}
