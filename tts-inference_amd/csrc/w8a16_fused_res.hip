// The W8A16 skinny kernel with the residual add in its epilogue, for 1 to 8 staged
// decode rows: `hidden = residual + o_proj(...)` and `hidden + down(...)`
// (qtts/models/talker.py:270-271) as one launch.  Kept apart from w8a16_fused.hip so
// the two instantiation sets compile in parallel.
#include "skinny_fused.h"

namespace qtts {

template int launch_fused<kProNone, true, 1>(int, bool, const FusedArgs&);
template int launch_fused<kProNone, true, 2>(int, bool, const FusedArgs&);
template int launch_fused<kProNone, true, 4>(int, bool, const FusedArgs&);
template int launch_fused<kProNone, true, 8>(int, bool, const FusedArgs&);

}  // namespace qtts
