// Error reporting shared by the translation units of libmt_attn.so: every C
// entry point returns 0 or a code, and records a message for mt_last_error()
// on failure (per calling thread).
#pragma once

namespace mt_abi {

__attribute__((visibility("hidden"))) int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
__attribute__((visibility("hidden"))) int ok();
__attribute__((visibility("hidden"))) const char* last_error();
// Compute units of the current device (cached per device).
__attribute__((visibility("hidden"))) int device_cus();

}  // namespace mt_abi
