/*
 * The reference engine's translation unit (k3_engine.cu, with
 * k3_engine_prefill.inc) followed by the routed-MoE binding of libk3moe
 * (k3_engine_moe.inc), compiled as one unit: the binding is code a
 * maintainer would add to k3_engine.cu, so it is built against the engine's
 * own types and constants rather than restatements of them. Test code:
 * tests/engine_link/Makefile builds it; nothing under moonshine_amd/ uses it.
 */
#include "k3_engine.cu"
#include "k3_engine_moe.inc"
