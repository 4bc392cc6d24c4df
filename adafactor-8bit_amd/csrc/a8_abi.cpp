// Error state and version of the C ABI.
#include <string>

#include "a8_abi_impl.h"

namespace a8 {
static thread_local std::string g_err;
void set_error_msg(const char* msg) { g_err = msg ? msg : ""; }
}  // namespace a8

extern "C" const char* a8_last_error(void) { return a8::g_err.c_str(); }
extern "C" const char* a8_version(void) { return "adafactor8bit_amd 0.1.0 (gfx950)"; }
