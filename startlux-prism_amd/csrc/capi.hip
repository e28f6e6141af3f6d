// Library-level C ABI: version and error strings.
#include "common.h"

extern "C" int prism_version(void) { return 100; }

extern "C" const char* prism_error_string(int code) {
    switch (code) {
        case PRISM_OK: return "ok";
        case PRISM_ERR_SHAPE: return "unsupported shape";
        case PRISM_ERR_ALIGN: return "misaligned pointer or stride";
        case PRISM_ERR_ARG: return "bad argument";
        case PRISM_ERR_LAUNCH: return "kernel launch failed";
        case PRISM_ERR_DEVICE: return "the current device is not gfx950";
        default: return "unknown error";
    }
}
