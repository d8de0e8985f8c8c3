// capi_util.h -- error reporting shared by every extern "C" translation unit:
// functions return AIH_OK / AIH_ERR and leave the calling thread's message
// for aih_last_error(); no exception crosses the boundary
// (crates/ai-ffi/src/lib.rs:45-52,130-133).
#pragma once

#include <exception>
#include <string>

#include "../../include/aih_conv.h"

namespace aih {

// The calling thread's message for aih_last_error().
std::string &last_error_slot();

inline int api_fail(const std::string &msg) {
  last_error_slot() = msg;
  return AIH_ERR;
}

template <class F>
int api_guarded(F &&f) {
  try {
    return f();
  } catch (const std::exception &e) {
    return api_fail(std::string("exception: ") + e.what());
  } catch (...) {
    return api_fail("unknown exception");
  }
}

}  // namespace aih
