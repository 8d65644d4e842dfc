// GatedMLP's gate_up_proj with its activation in the epilogue (skinny.h: PAIR), for 1
// to 8 staged decode rows: silu(gate) * up written straight from the GEMM, the gate_up
// output never stored (qtts/layers/activation.py:142-147).
#include "skinny_fused.h"

namespace qtts {

template int launch_fused<kProNone, false, 1, true>(int, bool, const FusedArgs&);
template int launch_fused<kProNone, false, 2, true>(int, bool, const FusedArgs&);
template int launch_fused<kProNone, false, 4, true>(int, bool, const FusedArgs&);
template int launch_fused<kProNone, false, 8, true>(int, bool, const FusedArgs&);

}  // namespace qtts
