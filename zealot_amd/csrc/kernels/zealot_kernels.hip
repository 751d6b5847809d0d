// zealot_kernels.hip — the single gfx950 code object loaded by libzealot_hip
// with hipModuleLoad. Every kernel is extern "C" so the host looks it up by
// name; see gemm_mfma.hip, narrow.hip and ppo_kernels.hip.
#include "gemm_mfma.hip"
#include "narrow.hip"
#include "ppo_kernels.hip"
