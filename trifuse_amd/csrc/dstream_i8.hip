// The streaming decode kernels for 8-bit codes with bf16 storage
// (namespace tfm::ds_bf16_i8); the source is dstream.hip.
#define TFM_DS_BITS 8
#include "dstream.hip"
