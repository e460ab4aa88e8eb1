// ABI helpers of libdiffrast_hip.so: error strings, version and struct sizes.
#include "common.h"

extern "C" const char* dr_error_string(int code) {
  switch (code) {
    case DR_OK: return "success";
    case DR_ERR_ARGUMENT: return "invalid argument (a size, pointer or mode is out of range)";
    case DR_ERR_CAPACITY: return "workspace or buffer smaller than required";
    case DR_ERR_HIP: return hipGetErrorString(hipPeekAtLastError());
    case DR_ERR_SCRATCH:
      return "the call needs more memory than the 64 MiB static scratch buffer of the "
             "allocation-free entry point holds (its visibility workspace, "
             "dr_raster_workspace_size, must be at most 64 MiB - 32 KiB)";
    default: return "unknown error";
  }
}

extern "C" int dr_abi_version(void) { return 15; }

extern "C" int dr_struct_size(int which) {
  switch (which) {
    case 0: return (int)sizeof(DrRasterGeometry);
    case 1: return (int)sizeof(DrInterpolateArgs);
    case 2: return (int)sizeof(DrTextureArgs);
    case 3: return (int)sizeof(DrAntialiasArgs);
    default: return -1;
  }
}
