// The two-launch layer's kernels (fused.hip) compiled once more with per-workgroup clock stamps
// (FusedLayerParams::ts) and launchers named launch_fused_attn_timed / launch_fused_mlp_timed.
// Only qe_profile_step's in-step timing launches them; the decode path launches fused.hip's
// unstamped kernels, which read no clock.
#define QE_FUSED_TIMED 1
#include "fused.hip"
