// Library-level entry points of libshard_hip.so: version and error text.
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace shard {

static thread_local char g_last_error[256] = "";

void set_last_error(const char* what, hipError_t err) {
  snprintf(g_last_error, sizeof(g_last_error), "%s: %s (%d)", what, hipGetErrorString(err),
           (int)err);
}

void set_last_text(const char* text) { snprintf(g_last_error, sizeof(g_last_error), "%s", text); }

}  // namespace shard

extern "C" {

const char* shard_version(void) { return "shard_hip 0.1.0 gfx950"; }

const char* shard_last_error(void) { return shard::g_last_error; }

size_t shard_decode_args_size(void) { return sizeof(shard_decode_args); }

}  // extern "C"
