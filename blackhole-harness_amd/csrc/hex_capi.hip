// C-ABI plumbing of libbh_hex.so: per-thread error message, status helpers.
#include <string>

#include "hex_common.h"

namespace bh {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(BH_HEX_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return BH_HEX_OK;
}

}  // namespace bh

extern "C" {

const char* bh_hex_last_error(void) { return bh::g_last_error.c_str(); }

int bh_hex_abi_version(void) { return BH_HEX_ABI_VERSION; }

}  // extern "C"
