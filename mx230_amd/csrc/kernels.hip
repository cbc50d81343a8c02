// The gfx950 code object of libmxfa (mxfa_gfx950.hsaco): every device source
// in one translation unit, compiled for the device only; the kernels it
// exports are named in fa_kernels.h.
#include "fa_fwd.hip"
#include "fa_bwd.hip"
#include "fa_naive.hip"
#include "probe.hip"
