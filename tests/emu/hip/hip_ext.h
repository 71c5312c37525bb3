// Host stand-in for <hip/hip_ext.h>, used ONLY by tests/emu: the kernel
// headers include it for the launchers' profiling launches, which the CPU
// emulator does not compile (it calls the kernels itself).
#pragma once
#include "hip_runtime.h"
