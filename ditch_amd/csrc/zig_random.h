// zig_random.h — the random stream the reference draws from, on the host:
// Zig's std.Random.DefaultPrng (Xoshiro256++ whose 256-bit state is filled
// by SplitMix64 from the seed), Random.float(f64), and Random.floatNorm
// (Zig's ziggurat for N(0, 1) with 256 layers, r = 3.6541528853610088,
// v = 0.00492867323399). The reference uses it for the randomised SVD's test
// matrix (abliterate.zig:473-479), the sketch's test matrix
// (directions.zig:65-67) and the Sampler's draws (model.zig:5208-5262).
// This is the algorithm of Zig 0.16's lib/std/Random (Xoshiro256.zig,
// SplitMix64.zig, ziggurat.zig, Random.zig float), restated; the reference
// pins minimum_zig_version 0.16.0 (build.zig.zon).
#pragma once

#include <math.h>
#include <stdint.h>

namespace ditch {

struct ZigRandom {
    uint64_t s[4];

    static uint64_t splitmix_next(uint64_t &x) {
        x += 0x9e3779b97f4a7c15ull;
        uint64_t z = x;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

    ZigRandom() : s{0, 0, 0, 0} {}
    explicit ZigRandom(uint64_t seed) {
        uint64_t x = seed;
        for (int i = 0; i < 4; i++) s[i] = splitmix_next(x);
    }
    static ZigRandom from_state(const uint64_t st[4]) {
        ZigRandom r;
        for (int i = 0; i < 4; i++) r.s[i] = st[i];
        return r;
    }

    // Xoshiro256++ (Random.int(u64) is one step)
    uint64_t next() {
        const uint64_t r = rotl(s[0] + s[3], 23) + s[0];
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }

    // Random.float(f64): 52 mantissa bits from one draw, the exponent from
    // its leading zeros; when the top 12 bits are all zero, further draws
    // extend the leading-zero count (capped at 1022).
    double float64() {
        const uint64_t rand = next();
        uint64_t lz = rand ? (uint64_t)__builtin_clzll(rand) : 64;
        if (lz >= 12) {
            lz = 12;
            for (;;) {
                const uint64_t r2 = next();
                const uint64_t add = r2 ? (uint64_t)__builtin_clzll(r2) : 64;
                lz += add;
                if (add != 64) break;
                if (lz >= 1022) {
                    lz = 1022;
                    break;
                }
            }
        }
        const uint64_t bits = ((1022 - lz) << 52) | (rand & 0xFFFFFFFFFFFFFull);
        double d;
        __builtin_memcpy(&d, &bits, 8);
        return d;
    }

    struct NormTables {
        double x[257], f[257];
    };
    static constexpr double norm_r = 3.6541528853610088;
    static constexpr double norm_v = 0.00492867323399;
    static double norm_pdf(double x) { return exp(-x * x / 2.0); }
    static double norm_pdf_inv(double y) { return sqrt(-2.0 * log(y)); }
    static const NormTables &norm_tables() {
        static const NormTables t = [] {
            NormTables z;
            z.x[0] = norm_v / norm_pdf(norm_r);
            z.x[1] = norm_r;
            for (int i = 2; i < 256; i++) z.x[i] = norm_pdf_inv(norm_v / z.x[i - 1] + norm_pdf(z.x[i - 1]));
            z.x[256] = 0.0;
            for (int i = 0; i < 257; i++) z.f[i] = norm_pdf(z.x[i]);
            return z;
        }();
        return t;
    }

    // ziggurat.next_f64 over the normal tables: the low 8 bits of one draw
    // pick the layer, its top 52 bits a u in [-1, 1).
    double norm() {
        const NormTables &t = norm_tables();
        for (;;) {
            const uint64_t bits = next();
            const int i = (int)(bits & 0xff);
            const uint64_t repr = (0x400ull << 52) | (bits >> 12);
            double u;
            __builtin_memcpy(&u, &repr, 8);
            u -= 3.0;
            const double x = u * t.x[i];
            if (fabs(x) < t.x[i + 1]) return x;
            if (i == 0) {  // the tail beyond r
                double tx = 1.0, ty = 0.0;
                while (-2.0 * ty < tx * tx) {
                    tx = log(float64()) / norm_r;
                    ty = log(float64());
                }
                return u < 0 ? tx - norm_r : norm_r - tx;
            }
            if (t.f[i + 1] + (t.f[i] - t.f[i + 1]) * float64() < norm_pdf(x)) return x;
        }
    }

    // Random.floatNorm(f32): the f64 draw rounded to f32
    float norm_f32() { return (float)norm(); }
};

}  // namespace ditch
