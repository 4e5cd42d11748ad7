// cuca_kernels.hip -- the one gfx950 code object of the library.
//
// Built with: hipcc --offload-arch=gfx950 --offload-device-only
//   --no-gpu-bundle-output -O3 -ffp-contract=off
//   -Xclang -target-feature -Xclang -packed-fp32-ops
// and embedded into libcuca_hip.so, which loads it with hipModuleLoadData
// and launches its extern "C" kernels with hipModuleLaunchKernel.
#include "embed.hip"
#include "norm.hip"
#include "glu.hip"
#include "rope.hip"
#include "attn.hip"
#include "qmm.hip"
#include "pick.hip"
#include "qmv.hip"
#include "qmd.hip"
#include "qgemm.hip"
#include "gemm16.hip"
#include "attn_rows.hip"
