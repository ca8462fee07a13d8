// Decode kernels instantiated for head_dim = 128 (all head tiles, FP16 and INT8).
#include "pa_decode_kernels.hpp"

namespace pa {
hipError_t launch_decode_d128(const DecodeLaunch& l) { return launch_decode_d<128>(l); }
int sched_groups_d128(int waves, bool int8_kv) { return sched_groups_d<128>(waves, int8_kv); }
}  // namespace pa
