// Host build of the kernels' exp / log (the same source as the device code),
// so that CPU tests can check them against the oracle without a GPU.
#include "otx_math.h"

extern "C" float otx_host_expf(float x) { return otx_expf(x); }
extern "C" float otx_host_logf(float x) { return otx_logf(x); }
extern "C" uint16_t otx_host_f32_to_bf16(float x) { return otx_f32_to_bf16(x); }
extern "C" float otx_host_div_rn(float a, float b) { return otx_div_rn(a, b); }
