/* CPU stand-in for <hip/hip_runtime.h>, used only to build the kernels for the SIMT emulator
 * (tests/cpu/simt/simt.h). Test infrastructure: never part of the product library. */
#pragma once
#include "../simt.h"
