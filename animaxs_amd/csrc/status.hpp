// Status codes, exceptions and the thread-local last-error message of the C ABI
// (the reference throws AnimapkError.validation(String),
// AnimaXS/Runtime/Animapk/MappedFile.swift:14).  No HIP dependency.
#pragma once

#include <new>
#include <stdexcept>
#include <string>

#include "anima_hip.h"

namespace anima {

struct Error : std::runtime_error {
  anima_status status;
  Error(anima_status s, const std::string& m) : std::runtime_error(m), status(s) {}
};

[[noreturn]] inline void fail(anima_status s, const std::string& msg) { throw Error(s, msg); }

void set_last_error(const char* msg);

// Runs f, converting exceptions into a status code + thread-local message.
template <class F>
anima_status guarded(F&& f) {
  try {
    f();
    set_last_error("");
    return ANIMA_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.status;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return ANIMA_E_DEVICE;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return ANIMA_E_DEVICE;
  }
}

}  // namespace anima
