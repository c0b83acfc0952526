// Single translation unit for the gfx950 code object: every kernel of the
// library, resolved by name through hipModuleGetFunction.
#include "quantize.hip"
#include "gemv.hip"
#include "gemm.hip"
#include "gemm_f32.hip"
#include "moe.hip"
#include "gemm_persistent.hip"
