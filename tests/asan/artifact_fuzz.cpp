// Host-only robustness driver for the artifact reader of libtinyinfer_llm
// (tinyinfer_amd/csrc/artifact.hpp), built with AddressSanitizer and UBSan by
// tests/test_artifact_asan.py.  Every input must either be accepted or raise
// Invalid / IOError; a memory error or undefined behaviour aborts the process.
//
//   artifact_fuzz json FILE...      JsonReader(text).parse() on each file
//   artifact_fuzz manifest PATH...  load_artifact(path) on each manifest
//
// Prints "<accepted> <rejected>" and one line per accepted input.
#include <algorithm>
#include <cstdio>
#include <string>

#include "../../tinyinfer_amd/csrc/artifact.hpp"

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  const std::string mode = argv[1];
  int accepted = 0, rejected = 0;
  for (int i = 2; i < argc; ++i) {
    try {
      if (mode == "json") {
        const std::vector<uint8_t> raw = tia::art::read_file(argv[i], 1u << 20);
        const std::string text(raw.begin(), raw.end());
        (void)tia::art::JsonReader(text).parse();
      } else {
        const tia::art::Artifact a = tia::art::load_artifact(argv[i]);
        if (a.tensors.empty()) throw tia::art::Invalid("no tensors");
      }
      ++accepted;
      std::printf("accepted %s\n", argv[i]);
    } catch (const tia::art::Invalid&) {
      ++rejected;
    } catch (const tia::art::IOError&) {
      ++rejected;
    }
  }
  std::printf("%d %d\n", accepted, rejected);
  return 0;
}
