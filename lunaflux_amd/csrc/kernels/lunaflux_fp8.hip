// lunaflux_fp8.hip - the one translation unit of the gfx950 code object
// lunaflux_fp8.hsaco (hipcc --genco --offload-arch=gfx950).
#include "projection.hip"
#include "w8a16.hip"
#include "w8a16_gemm.hip"
#include "moe.hip"
#include "calibrate.hip"
