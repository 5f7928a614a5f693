// loader_tool -- the reference's Dataset / Loader (src/model_utils/
// dataset.cpp and loader.cpp, compiled where they lie by oracle/Makefile)
// on the fixed checks of tests/cpp/loader_tool_content.h.
// TEST INFRASTRUCTURE ONLY.
//   loader_tool TOKENS_FILE TEXT_FILE
#include "loader_tool_content.h"
#include "model_utils/Dataset.h"
#include "model_utils/loader.h"

int main(int argc, char **argv) {
  if (argc != 3) return 2;
  try {
    return loader_test_content::run<Dataset, Loader>(argv[1], argv[2]);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "loader_tool: %s\n", e.what());
    return 1;
  }
}
