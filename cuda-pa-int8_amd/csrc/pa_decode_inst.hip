// Decode kernels instantiated for one head_dim: this file is compiled once
// per supported head_dim with -DPA_HEAD_DIM=<D> (every kind, FP16 and INT8).
#include "pa_decode_kernels.hpp"

#ifndef PA_HEAD_DIM
#error "compile once per head_dim with -DPA_HEAD_DIM=<D>"
#endif

#define PA_CAT_(a, b) a##b
#define PA_CAT(a, b) PA_CAT_(a, b)

namespace pa {
hipError_t PA_CAT(launch_decode_d, PA_HEAD_DIM)(const DecodeLaunch& l) {
  return launch_decode_d<PA_HEAD_DIM>(l);
}
int PA_CAT(resident_groups_d, PA_HEAD_DIM)(bool stream_part, int waves, bool int8_kv,
                                            int column_tiles) {
  return resident_groups_d<PA_HEAD_DIM>(stream_part, waves, int8_kv, column_tiles);
}
}  // namespace pa
