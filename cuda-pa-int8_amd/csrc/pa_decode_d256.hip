// Decode kernels instantiated for head_dim = 256 (all head tiles, FP16 and INT8).
#include "pa_decode_kernels.hpp"

namespace pa {
hipError_t launch_decode_d256(const DecodeLaunch& l) { return launch_decode_d<256>(l); }
int sched_groups_d256(int waves, bool int8_kv) { return sched_groups_d<256>(waves, int8_kv); }
}  // namespace pa
