// zealot_kernels.hip — the single gfx950 code object loaded by libzealot_hip
// with hipModuleLoad. Every kernel is extern "C" so the host looks it up by
// name; see gemm_mfma.hip, narrow.hip, ppo_kernels.hip, head.hip and
// obs_norm.hip.
#include "gemm_mfma.hip"
#include "narrow.hip"
#include "obs_norm.hip"
#include "ppo_kernels.hip"
#include "head.hip"
#include "policy.hip"
