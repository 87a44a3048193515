/*
 * include/k3_rocm_ops.h against the reference's k3_rocm_ops.h (test code).
 * Both are included in one translation unit, the reference's first; the
 * include guard (the same name in both, as a drop-in header needs) is
 * lifted in between so every declaration of ours is read as a
 * redeclaration. A parameter or return type that differs from the
 * reference's is then a compile error, in C and in C++.
 */
#include REF_OPS_H
#undef K3_ROCM_OPS_H
#include OUR_OPS_H

int k3_header_compat_ok(void) { return 1; }
