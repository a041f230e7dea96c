// The streaming decode kernels for IEEE-half activations, scales and biases
// (namespace tfm::ds_f16); the source is dstream.hip.
#define TFM_DS_F16 1
#include "dstream.hip"
