// Checker-only driver: exposes the reference's CPU query-RoPE (src/q_rope.h:3-35,
// `rope_cpu`) through a C symbol so tests can compare the oracle's rotation with it.
// Built by oracle/Makefile into oracle/_ref/ from the reference sources where they
// lie; nothing here is part of the product.
#include "q_rope.h"

extern "C" void ref_rope_cpu_f32(float* rotated_queries, const float* queries, const float* cosines,
                                 const float* sines, int F, int W, int Hq, int S, int E, int RotaryE) {
    rope_cpu<float>(rotated_queries, queries, cosines, sines, F, W, Hq, S, E, RotaryE);
}
