// smoe_api.cpp — status strings and version of the smoe C ABI.
#include "../../include/smoe.h"

extern "C" const char* smoe_strerror(int status) {
  switch (status) {
    case SMOE_OK: return "ok";
    case SMOE_EINVAL_NULL: return "smoe: a required pointer is NULL";
    case SMOE_EINVAL_DIM: return "smoe: a dimension is non-positive or out of range";
    case SMOE_EINVAL_ALIGN128: return "smoe: H / I / N / Kdim must be a multiple of 128";
    case SMOE_EINVAL_EXPERTS: return "smoe: expert count must be in [1, 1024]";
    case SMOE_EINVAL_WORKSPACE: return "smoe: workspace missing or too small";
    case SMOE_EINVAL_PTRALIGN: return "smoe: pointer not 16-byte aligned";
    case SMOE_EINVAL_TOPK: return "smoe: top-k must be in [1, min(E, 32)]";
    case SMOE_EINVAL_MODE: return "smoe: mode argument out of range";
    default: return status > 0 ? "smoe: HIP error (value is a hipError_t)" : "smoe: unknown error";
  }
}

extern "C" const char* smoe_version(void) { return "smoe 0.1 gfx950"; }
