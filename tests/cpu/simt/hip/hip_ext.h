/* CPU stand-in for <hip/hip_ext.h>, used only to build the kernels for the SIMT emulator
 * (tests/cpu/simt/simt.h defines hipExtLaunchKernelGGL). Test infrastructure: never part of the product library. */
#pragma once
#include "../simt.h"
