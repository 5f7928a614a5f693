// test_loader -- templit_amd's Dataset / Loader on the fixed checks of
// loader_tool_content.h, for comparison with the reference's
// (oracle/loader_tool.cpp). Host only, no GPU.
//   test_loader TOKENS_FILE TEXT_FILE
#include "loader_tool_content.h"
#include "model_utils/Dataset.h"
#include "model_utils/loader.h"

int main(int argc, char **argv) {
  if (argc != 3) return 2;
  try {
    return loader_test_content::run<Dataset, Loader>(argv[1], argv[2]);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "test_loader: %s\n", e.what());
    return 1;
  }
}
