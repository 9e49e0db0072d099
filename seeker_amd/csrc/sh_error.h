// Error reporting shared by the host code of libseeker_hip (no HIP headers):
// a failing call stores a message for sh_last_error() and returns a status.
#pragma once
#include "../../include/seeker_hip.h"

void sh_set_error(const char* fmt, ...);

#define SH_CHECK(cond, code, ...) \
  do {                            \
    if (!(cond)) {                \
      sh_set_error(__VA_ARGS__);  \
      return (code);              \
    }                             \
  } while (0)
