// zi_sample_cap.hip -- the final-logit softcap instances of the sampling
// kernels (src/model.zig:2492-2510 fused into the read), compiled apart from
// the uncapped ones so that those carry no softcap code.
#define ZI_SAMPLE_CAP 1
#include "zi_sample.hip"
