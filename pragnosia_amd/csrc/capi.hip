// Library-level entry points: ABI version and return-code names.
#include "common.h"

extern "C" int pragnosia_abi_version(void) { return 22; }

extern "C" const char* pragnosia_error_string(int code) {
  if (code == PRAGNOSIA_OK) return "ok";
  if (code == PRAGNOSIA_ERR_INVALID_ARGUMENT) return "invalid argument (shape, pointer or option rejected)";
  if (code == PRAGNOSIA_ERR_UNSUPPORTED) return "unsupported configuration";
  if (code == PRAGNOSIA_ERR_TOO_LARGE) return "shape needs more scratch than the allocation-free entry point holds";
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown error";
}
