// Launchers whose gfx950 kernels are not built yet answer UNAVAILABLE.
#include "kernels.hpp"

namespace pih_amd {
St LaunchFp4Gemm(const Fp4GemmArgs&) { return Unavailable("fp4_gemm_not_built"); }
St LaunchBf16Gemm(const Bf16GemmArgs&) { return Unavailable("bf16_gemm_not_built"); }
uint64_t Bf16GemmWorkspaceBytes(uint32_t, uint32_t, uint32_t) { return 0; }
St LaunchW4a16(const W4a16Args&) { return Unavailable("w4a16_not_built"); }
uint64_t W4a16WorkspaceBytes(uint32_t, uint32_t, uint32_t) { return 0; }
}  // namespace pih_amd
