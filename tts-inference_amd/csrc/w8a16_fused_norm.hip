// The W8A16 skinny kernel with the RMSNorm prologue for 2 to 8 staged decode rows:
// `qkv_proj(input_layernorm(hidden))` and `gate_up_proj(post_attention_layernorm(...))`
// (qtts/models/talker.py:246-271) as one launch at batch sizes above one.  Kept
// apart from w8a16_fused.hip so the instantiation sets compile in parallel.
#include "skinny_fused.h"

namespace qtts {

template int launch_fused<kProRmsNorm, false, 2>(int, bool, const FusedArgs&);
template int launch_fused<kProRmsNorm, false, 4>(int, bool, const FusedArgs&);
template int launch_fused<kProRmsNorm, false, 8>(int, bool, const FusedArgs&);

}  // namespace qtts
