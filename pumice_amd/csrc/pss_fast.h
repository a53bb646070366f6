/* pss_fast.h - register-resident segmented sampler kernel (in progress). */
#ifndef PSS_FAST_H
#define PSS_FAST_H
#include "pss_device.h"
static inline size_t pss_fast_ws_bytes(uint32_t V, uint32_t rows) { (void)V; (void)rows; return 0; }
static inline int pss_fast_supported(uint32_t V, uint32_t dtype, uint32_t rows) { (void)V; (void)dtype; (void)rows; return 0; }
static inline hipError_t pss_fast_launch(const pss_args& a, uint32_t rows, hipStream_t st) { (void)a; (void)rows; (void)st; return hipErrorNotSupported; }
#endif
