// The streaming decode kernels for 8-bit codes with IEEE-half storage
// (namespace tfm::ds_f16_i8); the source is dstream.hip.
#define TFM_DS_F16 1
#define TFM_DS_BITS 8
#include "dstream.hip"
