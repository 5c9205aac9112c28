"""MI355X (gfx950) implementation of slotstream-spark's MTP verify path: the affine-4bit routed MoE layer
(router, slot-table lookup, gate/up with in-register dequant, SwiGLU, down, rank-order combine, shared expert)
and greedy / p-q acceptance. Hand-written HIP kernels behind the C ABI of include/ssmoe.h (libssmoe.so)."""
