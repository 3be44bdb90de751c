// gen.cpp - seeded synthetic inputs for the five benchmark configurations.
//
// The reference benchmarks SuiteSparse files (`cant`, `ASIC_320k`) that are
// not available offline; these generators produce matrices of the shapes the
// benchmark configurations describe.  Every random stream is a splitmix64
// sequence (Steele, Lea & Flood, "Fast splittable pseudorandom number
// generators", OOPSLA 2014) keyed by (seed, config tag, row or block-row), so
// rows can be generated in parallel and the output depends only on the seed.
//   uniform value : 24 high bits -> (u - 2^23) * 2^-23, in [-1, 1)
//   normal value  : Box-Muller in double, narrowed to float
//   integer < n   : (32 high bits * n) >> 32
//
//   cfg1  4,096^2, exactly 16 distinct uniform columns per row, U[-1,1).
//   cfg2  62,451^2 banded FEM-like: 20,817 block-rows of 3x3 dense blocks,
//         symmetric (blocks and values mirrored).  Block-row I picks upper
//         blocks among I+1..I+333 (band half-width 999 columns) so that its
//         block count reaches a target drawn from 17..25, never letting a
//         block-row exceed 26 blocks; block-rows are processed in order, so
//         lower blocks come from earlier picks.  nnz/row lies in [51, 78],
//         mean ~63, ~3.94M nnz.  Off-diagonal values N(0,1); each diagonal
//         entry is the row's off-diagonal l1 norm + 1 (diagonally dominant).
//   cfg3  321,821^2 circuit-like power law: row r draws k off-diagonal
//         columns, k ~ Zipf(alpha=2) on [1, 60000]; each draw is r+U{-64..64}
//         (clamped) with probability 0.7, else U[0,M).  Columns are deduped
//         and the diagonal is added.  ~1.86M nnz, longest row ~13-18k.
//   cfg4  10^6 x 10^6, exactly 16 distinct uniform columns per row, U[-1,1).
//   cfg5  16,384^2 block-sparse: 1,024 block-rows, each with 51 distinct
//         uniform block-columns (5% of 1,024) of dense 16x16 N(0,1) blocks.
// COO entries come out row by row; within a row, columns are in draw order
// for cfg1/cfg4 and ascending for cfg2/cfg3/cfg5.
#include <algorithm>
#include <cmath>
#include <numeric>
#include <string>

#include "core.hpp"
#include "parallel.hpp"

namespace vcsr {
namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

struct Rng {
    uint64_t s;
    uint64_t next() {
        s += 0x9E3779B97F4A7C15ULL;
        return mix64(s);
    }
    // Integer in [0, n), n < 2^32.
    uint32_t below(uint32_t n) { return (uint32_t)(((next() >> 32) * (uint64_t)n) >> 32); }
    float uniform() { return (float)((int32_t)(next() >> 40) - (1 << 23)) * (1.0f / 8388608.0f); }
    double unit_open() { return ((double)(next() >> 11) + 1.0) * (1.0 / 9007199254740992.0); }
    double unit() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
    float normal() {
        const double u1 = unit_open(), u2 = unit();
        return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
};

inline Rng stream(uint64_t seed, uint64_t tag, uint64_t idx) {
    return Rng{mix64(seed + 0x632BE59BD9B4E019ULL * (tag + 1)) ^
               mix64(idx * 0x9E3779B97F4A7C15ULL + 0xD1B54A32D192ED03ULL)};
}

// Rows with exactly `per_row` distinct uniform columns (cfg1, cfg4).
Coo gen_uniform_rows(int32_t M, int32_t N, int per_row, uint64_t seed, uint64_t tag) {
    Coo coo;
    coo.M = M;
    coo.N = N;
    const size_t nnz = (size_t)M * per_row;
    coo.rows.resize(nnz);
    coo.cols.resize(nnz);
    coo.vals.resize(nnz);
    parallel_for(M, 8192, default_threads(), [&](int64_t rb, int64_t re) {
        for (int64_t r = rb; r < re; ++r) {
            Rng g = stream(seed, tag, (uint64_t)r);
            int32_t* c = coo.cols.data() + (size_t)r * per_row;
            for (int i = 0; i < per_row; ++i) {
                for (;;) {
                    const int32_t x = (int32_t)g.below((uint32_t)N);
                    bool dup = false;
                    for (int j = 0; j < i; ++j) dup |= (c[j] == x);
                    if (!dup) { c[i] = x; break; }
                }
            }
            for (int i = 0; i < per_row; ++i) {
                coo.rows[(size_t)r * per_row + i] = (int32_t)r;
                coo.vals[(size_t)r * per_row + i] = g.uniform();
            }
        }
    });
    return coo;
}

Coo gen_banded(uint64_t seed) {
    const int32_t nb = 20817, W = 333, cap = 26;
    const int32_t M = 3 * nb;
    std::vector<int32_t> cnt((size_t)nb, 1);
    std::vector<std::vector<int32_t>> upper((size_t)nb);
    std::vector<int32_t> cand;
    for (int32_t I = 0; I < nb; ++I) {
        Rng g = stream(seed, 2, (uint64_t)I);
        const int32_t target = 17 + (int32_t)g.below(9);
        const int32_t need = target - cnt[I];
        if (need <= 0) continue;
        cand.clear();
        for (int32_t J = I + 1; J <= std::min(I + W, nb - 1); ++J)
            if (cnt[J] < cap) cand.push_back(J);
        const int32_t k = std::min<int32_t>(need, (int32_t)cand.size());
        for (int32_t i = 0; i < k; ++i) {  // partial Fisher-Yates
            const int32_t j = i + (int32_t)g.below((uint32_t)(cand.size() - i));
            std::swap(cand[i], cand[j]);
        }
        std::sort(cand.begin(), cand.begin() + k);
        for (int32_t i = 0; i < k; ++i) {
            upper[I].push_back(cand[i]);
            cnt[cand[i]]++;
        }
        cnt[I] += k;
    }
    // Block lists per block-row: lower (mirrors), diagonal, upper; ascending.
    std::vector<std::vector<int32_t>> lower((size_t)nb);
    for (int32_t I = 0; I < nb; ++I)
        for (int32_t J : upper[I]) lower[J].push_back(I);
    // Upper block values: 9 per block, from block-row I's value stream;
    // diagonal block: 3 off-diagonal values (01, 02, 12).
    std::vector<int64_t> uoff((size_t)nb + 1, 0);
    for (int32_t I = 0; I < nb; ++I) uoff[I + 1] = uoff[I] + (int64_t)upper[I].size();
    std::vector<float> uval((size_t)uoff[nb] * 9), dval((size_t)nb * 3);
    parallel_for(nb, 1024, default_threads(), [&](int64_t ib, int64_t ie) {
        for (int64_t I = ib; I < ie; ++I) {
            Rng g = stream(seed, 3, (uint64_t)I);
            for (int q = 0; q < 3; ++q) dval[(size_t)I * 3 + q] = g.normal();
            for (int64_t u = uoff[I] * 9; u < uoff[I + 1] * 9; ++u) uval[(size_t)u] = g.normal();
        }
    });
    // Position of block (I,J) among upper[I], for mirrored lookups.
    auto upper_index = [&](int32_t I, int32_t J) -> int64_t {
        const auto& v = upper[I];
        return uoff[I] + (int64_t)(std::lower_bound(v.begin(), v.end(), J) - v.begin());
    };
    Coo coo;
    coo.M = M;
    coo.N = M;
    int64_t nnz = 0;
    for (int32_t I = 0; I < nb; ++I) nnz += 9 * (int64_t)cnt[I];
    coo.rows.reserve((size_t)nnz);
    coo.cols.reserve((size_t)nnz);
    coo.vals.reserve((size_t)nnz);
    for (int32_t I = 0; I < nb; ++I) {
        for (int a = 0; a < 3; ++a) {
            const int32_t r = 3 * I + a;
            const size_t row_begin = coo.vals.size();
            size_t diag_pos = 0;
            double l1 = 0.0;
            auto put = [&](int32_t c, float v) {
                coo.rows.push_back(r);
                coo.cols.push_back(c);
                coo.vals.push_back(v);
            };
            for (int32_t J : lower[I]) {  // A[3I+a][3J+b] = A[3J+b][3I+a] = upper(J,I)[b][a]
                const int64_t u = upper_index(J, I);
                for (int b = 0; b < 3; ++b) {
                    const float v = uval[(size_t)u * 9 + b * 3 + a];
                    l1 += std::fabs((double)v);
                    put(3 * J + b, v);
                }
            }
            for (int b = 0; b < 3; ++b) {
                if (a == b) {
                    diag_pos = coo.vals.size();
                    put(3 * I + b, 0.f);
                    continue;
                }
                const int lo = std::min(a, b), hi = std::max(a, b);
                const int q = (lo == 0) ? (hi - 1) : 2;  // 01->0, 02->1, 12->2
                const float v = dval[(size_t)I * 3 + q];
                l1 += std::fabs((double)v);
                put(3 * I + b, v);
            }
            for (size_t k = 0; k < upper[I].size(); ++k) {
                const int32_t J = upper[I][k];
                const int64_t u = uoff[I] + (int64_t)k;
                for (int b = 0; b < 3; ++b) {
                    const float v = uval[(size_t)u * 9 + a * 3 + b];
                    l1 += std::fabs((double)v);
                    put(3 * J + b, v);
                }
            }
            coo.vals[diag_pos] = (float)(l1 + 1.0);
            (void)row_begin;
        }
    }
    return coo;
}

Coo gen_powerlaw(uint64_t seed) {
    const int32_t M = 321821, kmax = 60000;
    // Zipf(2) on [1, kmax] by inverse CDF.
    std::vector<double> cdf((size_t)kmax);
    double acc = 0.0;
    for (int32_t k = 1; k <= kmax; ++k) {
        acc += 1.0 / ((double)k * (double)k);
        cdf[(size_t)k - 1] = acc;
    }
    for (auto& x : cdf) x /= acc;
    std::vector<std::vector<int32_t>> cols((size_t)M);
    std::vector<std::vector<float>> vals((size_t)M);
    parallel_for(M, 4096, default_threads(), [&](int64_t rb, int64_t re) {
        for (int64_t r = rb; r < re; ++r) {
            Rng g = stream(seed, 4, (uint64_t)r);
            const double u = g.unit();
            int32_t k = (int32_t)(std::lower_bound(cdf.begin(), cdf.end(), u) - cdf.begin()) + 1;
            if (k > kmax) k = kmax;
            auto& c = cols[(size_t)r];
            c.reserve((size_t)k + 1);
            for (int32_t i = 0; i < k; ++i) {
                int64_t x;
                if (g.below(10) < 7) {
                    x = r + (int64_t)g.below(129) - 64;
                    x = std::min<int64_t>(std::max<int64_t>(x, 0), M - 1);
                } else {
                    x = g.below((uint32_t)M);
                }
                c.push_back((int32_t)x);
            }
            c.push_back((int32_t)r);
            std::sort(c.begin(), c.end());
            c.erase(std::unique(c.begin(), c.end()), c.end());
            auto& v = vals[(size_t)r];
            v.resize(c.size());
            for (auto& x : v) x = g.uniform();
        }
    });
    Coo coo;
    coo.M = M;
    coo.N = M;
    size_t nnz = 0;
    for (const auto& c : cols) nnz += c.size();
    coo.rows.reserve(nnz);
    coo.cols.reserve(nnz);
    coo.vals.reserve(nnz);
    for (int32_t r = 0; r < M; ++r) {
        for (size_t i = 0; i < cols[(size_t)r].size(); ++i) {
            coo.rows.push_back(r);
            coo.cols.push_back(cols[(size_t)r][i]);
            coo.vals.push_back(vals[(size_t)r][i]);
        }
    }
    return coo;
}

Coo gen_blocksparse(uint64_t seed) {
    const int32_t nbr = 1024, bs = 16, per = 51;
    const int32_t M = nbr * bs;
    Coo coo;
    coo.M = M;
    coo.N = M;
    const size_t nnz = (size_t)nbr * per * bs * bs;
    coo.rows.resize(nnz);
    coo.cols.resize(nnz);
    coo.vals.resize(nnz);
    parallel_for(nbr, 16, default_threads(), [&](int64_t ib, int64_t ie) {
        std::vector<int32_t> bc(per);
        std::vector<float> blk((size_t)per * bs * bs);
        for (int64_t I = ib; I < ie; ++I) {
            Rng g = stream(seed, 5, (uint64_t)I);
            for (int i = 0; i < per; ++i) {
                for (;;) {
                    const int32_t x = (int32_t)g.below((uint32_t)nbr);
                    bool dup = false;
                    for (int j = 0; j < i; ++j) dup |= (bc[j] == x);
                    if (!dup) { bc[i] = x; break; }
                }
            }
            std::sort(bc.begin(), bc.end());
            for (auto& x : blk) x = g.normal();
            size_t o = (size_t)I * per * bs * bs;
            for (int a = 0; a < bs; ++a) {
                for (int i = 0; i < per; ++i) {
                    for (int b = 0; b < bs; ++b) {
                        coo.rows[o] = (int32_t)(I * bs + a);
                        coo.cols[o] = bc[i] * bs + b;
                        coo.vals[o] = blk[((size_t)i * bs + a) * bs + b];
                        ++o;
                    }
                }
            }
        }
    });
    return coo;
}

}  // namespace

Coo gen_coo(int cfg, uint64_t seed) {
    switch (cfg) {
        case 1: return gen_uniform_rows(4096, 4096, 16, seed, 1);
        case 2: return gen_banded(seed);
        case 3: return gen_powerlaw(seed);
        case 4: return gen_uniform_rows(1000000, 1000000, 16, seed, 6);
        case 5: return gen_blocksparse(seed);
        default: throw Error(1, "unknown synthetic config " + std::to_string(cfg));
    }
}

void gen_dense(uint64_t seed, int dist, int64_t rows, int32_t cols, float* out) {
    if (rows < 0 || cols < 0) throw Error(1, "negative dense shape");
    if (dist != 0 && dist != 1) throw Error(1, "dist must be 0 (uniform) or 1 (normal)");
    if (rows * (int64_t)cols > 0 && out == nullptr) throw Error(1, "null output buffer");
    const int64_t n = rows * (int64_t)cols;
    const uint64_t base = mix64(seed ^ 0xB5AD4ECEDA1CE2A9ULL);
    parallel_for(n, 1 << 16, default_threads(), [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; ++i) {
            if (dist == 0) {
                const uint64_t x = mix64(base + (uint64_t)i * 0x9E3779B97F4A7C15ULL);
                out[i] = (float)((int32_t)(x >> 40) - (1 << 23)) * (1.0f / 8388608.0f);
            } else {
                Rng g{base + (uint64_t)i * 0x3C6EF372FE94F82AULL};
                out[i] = g.normal();
            }
        }
    });
}

}  // namespace vcsr
