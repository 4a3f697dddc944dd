/* ORACLE — test infrastructure only. Force-included (-include) into the reference's engine
 * sources when they are compiled for oracle/_ref/libpinfer_refq4k.so: after <math.h>, the
 * DeltaNet gates' expf / log1pf (engine/src/forward_lin.c:18-19,59-66) name the oracle's
 * binary64-evaluated versions, which the device kernels also use. */
#ifndef ORC_GATE_LIBM_H
#define ORC_GATE_LIBM_H
#include <math.h>
float orc_gate_expf(float x);
float orc_gate_log1pf(float x);
#define expf orc_gate_expf
#define log1pf orc_gate_log1pf
#endif
