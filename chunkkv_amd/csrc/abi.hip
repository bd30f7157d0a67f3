// Library metadata entry points.
#include "ckv_common.hpp"

extern "C" int32_t ckv_abi_version(void) { return CKV_ABI_VERSION; }

extern "C" const char* ckv_status_string(int32_t status) {
  switch (status) {
    case CKV_OK: return "ok";
    case CKV_ERR_INVALID_ARGUMENT: return "invalid argument";
    case CKV_ERR_OUT_OF_RANGE: return "size or index out of range";
    case CKV_ERR_TOO_LARGE: return "request exceeds kernel capacity";
    case CKV_ERR_HIP: return "HIP launch error";
    default: return "unknown status";
  }
}
