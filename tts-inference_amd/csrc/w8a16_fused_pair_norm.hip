// post_attention_layernorm, gate_up_proj and GatedMLP's activation in one skinny
// launch (skinny.h: kProRmsNorm with PAIR), for 1 to 8 staged decode rows
// (qtts/models/talker.py:271 with qtts/layers/activation.py:142-147).
#include "skinny_fused.h"

namespace qtts {

template int launch_fused<kProRmsNorm, false, 1, true>(int, bool, const FusedArgs&);
template int launch_fused<kProRmsNorm, false, 2, true>(int, bool, const FusedArgs&);
template int launch_fused<kProRmsNorm, false, 4, true>(int, bool, const FusedArgs&);
template int launch_fused<kProRmsNorm, false, 8, true>(int, bool, const FusedArgs&);

}  // namespace qtts
