// dec_m0_h2.hip -- decode-shaped flash attention instantiations: unmasked, kv heads paired.
#include "fa_decode_inst.h"

namespace cvattn {
CVATTN_DECODE_PICK(fa_pick_decode_m0_h2, false, 2)
} // namespace cvattn
