// Runs the checkpoint header reader (csrc/safetensors.cpp) over the files
// named on the command line, for tests/test_sanitizers.py's ASan/UBSan build:
// prints "ok <tensors>" or "rejected <reason>" per file.
#include <cstdio>
#include <exception>

#include "safetensors.h"

int main(int argc, char** argv) {
  for (int i = 1; i < argc; ++i) {
    try {
      const hb::SafeFile f = hb::read_safetensors_header(argv[i]);
      std::printf("ok %zu\n", f.tensors.size());
    } catch (const std::exception& e) {
      std::printf("rejected %s\n", e.what());
    }
  }
  return 0;
}
