// The single gfx950 code object: every hot-path kernel in one translation
// unit, built with `hipcc --genco --offload-arch=gfx950` and loaded at run
// time by the module loader in g950rt.cpp.
#include "rowreduce.hip"
#include "gemm.hip"
#include "attention.hip"
#include "dequant.hip"
