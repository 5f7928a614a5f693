// test_loader -- templit_amd's Dataset / Loader on the fixed checks of
// loader_tool_content.h, for comparison with the reference's
// (oracle/loader_tool.cpp). Host only, no GPU.
//   test_loader TOKENS_FILE TEXT_FILE
//   test_loader --text-to-tokens TEXT_FILE OUT_FILE   (Dataset::load_text
//       with fraction 0.5, saved in the .tokens format)
#include "loader_tool_content.h"
#include "model_utils/Dataset.h"
#include "model_utils/loader.h"

#include <cstring>
#include <fstream>

int main(int argc, char **argv) {
  try {
    if (argc == 4 && std::strcmp(argv[1], "--text-to-tokens") == 0) {
      std::ifstream in(argv[2], std::ios::binary);
      const Dataset d = Dataset::load_text(in, 0.5);
      std::ofstream out(argv[3], std::ios::binary);
      d.save(out);
      return 0;
    }
    if (argc != 3) return 2;
    return loader_test_content::run<Dataset, Loader>(argv[1], argv[2]);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "test_loader: %s\n", e.what());
    return 1;
  }
}
