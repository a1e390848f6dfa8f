// Library-level entry points: error strings and ABI version.
#include "common.h"

extern "C" const char* face_hip_error_string(int code) {
    switch (code) {
        case 0: return "success";
        case FACE_ERR_ARG: return "invalid argument (shape, stride or null pointer)";
        case FACE_ERR_UNSUPPORTED: return "shape outside the instantiated kernel variants";
        case FACE_ERR_CAPACITY: return "row or bin capacity exceeded";
        case FACE_ERR_SCRATCH: return "input exceeds the fixed scratch of an allocation-free entry point";
        default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
    }
}

extern "C" int face_hip_abi_version(void) { return 24; }
