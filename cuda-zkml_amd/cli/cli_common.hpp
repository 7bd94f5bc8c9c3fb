// Shared helpers of the command-line front ends (zkml-prove, zkml-verify).
#pragma once
#include <stdio.h>
#include <string.h>

#include <chrono>
#include <string>

#include "zkml_gpu.h"

namespace cli {

inline const char* arg_value(int argc, char** argv, int& i) {
  if (i + 1 >= argc) {
    fprintf(stderr, "Error: %s needs a value\n", argv[i]);
    return nullptr;
  }
  return argv[++i];
}

struct Timer {
  std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
  double ms() const {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  }
};

inline const char* status_text(int st) { return zk_status_string(st); }

}  // namespace cli
