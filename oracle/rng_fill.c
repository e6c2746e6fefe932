/* Julia's Xoshiro stream and STADE's Box-Muller normals, as array fills --
 * TEST INFRASTRUCTURE ONLY (the checker's input generator; see oracle/rng.py).
 *
 * The same draws as oracle/rng.py's scalar loop, in C for the large inputs of the
 * full-size parity tests:
 *   rand(rng)      = (xoshiro256++ next >> 11) * 2^-53      (Julia's Float64 sampler)
 *   val_normal(rng) = sqrt(-2 log(1 - rand)) * cos(2 pi rand)
 *                    (/root/reference/src/STADE.jl:16628-16637, cosine branch)
 * Built with -ffp-contract=off; log and cos are the same libm the Python restatement
 * calls, and sqrt is correctly rounded in both, so the fills are bit-identical to the
 * scalar loop (tests/test_oracle_rng.py checks that).
 *
 * The state s[4] is read on entry and written back on exit, so a caller can continue the
 * stream in Python or in another fill.
 */
#include <math.h>
#include <stdint.h>

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static inline uint64_t next_u64(uint64_t s[4]) {
    uint64_t res = rotl(s[0] + s[3], 23) + s[0];
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return res;
}

static inline double rand01(uint64_t s[4]) { return (double)(next_u64(s) >> 11) * 0x1.0p-53; }

void oracle_rng_normal(uint64_t state[4], double* out, int64_t n) {
    uint64_t s[4] = {state[0], state[1], state[2], state[3]};
    const double two_pi = 2.0 * 3.141592653589793;
    for (int64_t i = 0; i < n; ++i) {
        double u1 = 1.0 - rand01(s);
        double u2 = rand01(s);
        out[i] = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    }
    for (int k = 0; k < 4; ++k) state[k] = s[k];
}

void oracle_rng_uniform(uint64_t state[4], double* out, int64_t n, double lo, double hi) {
    uint64_t s[4] = {state[0], state[1], state[2], state[3]};
    const double w = hi - lo;
    for (int64_t i = 0; i < n; ++i) out[i] = lo + w * rand01(s);
    for (int k = 0; k < 4; ++k) state[k] = s[k];
}
