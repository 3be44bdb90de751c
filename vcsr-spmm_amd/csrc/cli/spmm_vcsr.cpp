// spmm_vcsr - command-line driver of the gfx950 VCSR SpMM library.
//
// Flag surface of the reference harness (src/main.cpp:68-90):
//   --mtx F --O n --segw w --bundle b --tileK t --repeat r --algo X
// plus: --gen cfgN (synthetic BASELINE config instead of --mtx), --seed S,
// --layout H|S (VCSR builder for --algo vcsr), --warmup w, --check (L2 diff
// against the CPU CSR SpMM), --threads T (host threads), --expand-symmetric.
// Algorithms: csr (naive HIP CSR), vcsr (segmented streaming; aliases
// vcsr_baseline and vcsr_seg, the reference's names at main.cpp:135-146),
// vcsr_mfma (FP32-MFMA dense-block kernel on the same format), vcsr_tc
// (layout TC, segw=16 bundle=16, on the MFMA kernel), rocsparse (the vendor
// baseline; alias cusparse, the reference's name at main.cpp:119-123), aspt
// (wave-per-row CSR, the reference's ASpT competitor at main.cpp:153-157),
// fast (alias fastspmm: FastSpMM's fixed 16-row windows of condensed
// columns, main.cpp:158-162, on the FP32-MFMA tile kernel), cpu, all.
//
// Result lines keep the format of the published runs, which the reference's
// bench scripts parse (token before "ms" and before "GFLOP/s" on the last
// line; reports/a100/cant_O128_vcsr_segw4_b32_tk64.txt:3):
//   CSR (naive):   9.999 ms     52.10 GFLOP/s
//   VCSR (seg):    8.625 ms     60.40 GFLOP/s  [segw=4,bundle=32,tileK=64,groups=29825]
// Diagnostic lines (format build time, L2 diff, roofline) come before each
// result line so the last line of a single-algorithm run is the result.
#include <getopt.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../../include/vcsr_spmm.h"

namespace {

struct Opts {
    std::string mtx;
    int gen = 0;
    unsigned long long seed = 0;
    int O = 128, segw = 16, bundle = 64, tileK = 64, repeat = 10, warmup = 1;
    std::string algo = "all";
    std::string layout = "S";
    bool check = false;
    bool expand = false;
    int threads = 0;
    std::string save_fmt, load_fmt;  // VCSR format file for --algo vcsr
};

void usage() {
    std::printf("Usage: spmm_vcsr (--mtx file.mtx | --gen cfgN) --O 128 [options]\n");
    std::printf("Options: --segw w --bundle b --tileK t --repeat r --warmup w --seed s\n");
    std::printf("         --layout H|S --check --threads T --expand-symmetric\n");
    std::printf("         --save-fmt F (write the built VCSR format) --load-fmt F (use it\n");
    std::printf("         instead of building; --algo vcsr)\n");
    std::printf("Algorithms: csr, vcsr (vcsr_baseline, vcsr_seg), vcsr_mfma, vcsr_tc, "
                "rocsparse (cusparse), aspt, fast (fastspmm), cpu, all\n");
}

[[noreturn]] void die(const char* what, int rc) {
    std::fprintf(stderr, "spmm_vcsr: %s failed: %s\n", what, vcsr_last_error());
    std::exit(rc == VCSR_OK ? 1 : 2);
}

#define CHECK(call)                      \
    do {                                 \
        int rc_ = (call);                \
        if (rc_ != VCSR_OK) die(#call, rc_); \
    } while (0)

double now_ms() {
    return std::chrono::duration<double, std::milli>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

struct Check {
    double rel_l2 = 0, max_abs = 0, max_ratio = 0;
    bool ok = true;
};

// rel_L2 = ||C - R|| / ||R||; max-abs error of row r bounded by
// 1e-4 * ||A_r||_1 * max|B|.
Check compare(const std::vector<float>& C, const std::vector<float>& R,
              const std::vector<double>& row_l1, double bmax, int32_t O) {
    Check c;
    double num = 0, den = 0;
    const size_t M = row_l1.size();
    for (size_t r = 0; r < M; ++r) {
        const double tol = 1e-4 * row_l1[r] * bmax;
        for (int32_t k = 0; k < O; ++k) {
            const double d = (double)C[r * O + k] - (double)R[r * O + k];
            num += d * d;
            den += (double)R[r * O + k] * (double)R[r * O + k];
            const double a = std::fabs(d);
            c.max_abs = std::max(c.max_abs, a);
            if (tol > 0) c.max_ratio = std::max(c.max_ratio, a / tol);
            else if (a > 0) c.max_ratio = INFINITY;
        }
    }
    c.rel_l2 = den > 0 ? std::sqrt(num / den) : std::sqrt(num);
    c.ok = c.rel_l2 <= 1e-5 && c.max_ratio <= 1.0;
    return c;
}

}  // namespace

int main(int argc, char** argv) {
    Opts o;
    static struct option long_opts[] = {
        {"mtx", required_argument, 0, 'm'},    {"O", required_argument, 0, 'o'},
        {"segw", required_argument, 0, 's'},   {"bundle", required_argument, 0, 'b'},
        {"tileK", required_argument, 0, 't'},  {"repeat", required_argument, 0, 'r'},
        {"algo", required_argument, 0, 'a'},   {"gen", required_argument, 0, 'g'},
        {"seed", required_argument, 0, 'S'},   {"layout", required_argument, 0, 'L'},
        {"warmup", required_argument, 0, 'w'}, {"check", no_argument, 0, 'c'},
        {"threads", required_argument, 0, 'T'}, {"expand-symmetric", no_argument, 0, 'e'},
        {"save-fmt", required_argument, 0, 'F'}, {"load-fmt", required_argument, 0, 'l'},
        {"help", no_argument, 0, 'h'},         {0, 0, 0, 0}};
    int copt, idx;
    while ((copt = getopt_long(argc, argv, "", long_opts, &idx)) != -1) {
        switch (copt) {
            case 'm': o.mtx = optarg; break;
            case 'o': o.O = std::atoi(optarg); break;
            case 's': o.segw = std::atoi(optarg); break;
            case 'b': o.bundle = std::atoi(optarg); break;
            case 't': o.tileK = std::atoi(optarg); break;
            case 'r': o.repeat = std::atoi(optarg); break;
            case 'a': o.algo = optarg; break;
            case 'g': {
                const char* s = optarg;
                if (std::strncmp(s, "cfg", 3) == 0) s += 3;
                o.gen = std::atoi(s);
                break;
            }
            case 'S': o.seed = std::strtoull(optarg, nullptr, 10); break;
            case 'L': o.layout = optarg; break;
            case 'w': o.warmup = std::atoi(optarg); break;
            case 'c': o.check = true; break;
            case 'T': o.threads = std::atoi(optarg); break;
            case 'e': o.expand = true; break;
            case 'F': o.save_fmt = optarg; break;
            case 'l': o.load_fmt = optarg; break;
            case 'h': usage(); return 0;
            default: usage(); return 1;
        }
    }
    if (o.mtx.empty() == (o.gen == 0)) { usage(); return 1; }
    if (o.O <= 0 || o.repeat <= 0 || o.warmup < 0) { usage(); return 1; }
    if (o.algo == "vcsr_baseline" || o.algo == "vcsr_seg") o.algo = "vcsr";
    if (o.algo == "cusparse") o.algo = "rocsparse";
    if (o.algo == "fastspmm") o.algo = "fast";
    if (o.algo == "vcsr_naive") {
        std::printf("%s: not part of this build (vendor or competitor kernel)\n", o.algo.c_str());
        return 1;
    }
    const bool all = o.algo == "all";
    if (!all && o.algo != "csr" && o.algo != "vcsr" && o.algo != "vcsr_mfma" &&
        o.algo != "vcsr_tc" && o.algo != "rocsparse" && o.algo != "aspt" && o.algo != "fast" &&
        o.algo != "cpu") {
        usage();
        return 1;
    }
    const int layout = (o.layout == "H" || o.layout == "h") ? VCSR_LAYOUT_H : VCSR_LAYOUT_S;

    std::printf("=== VCSR-SpMM (MI355X gfx950) ===\n");
    vcsr_coo* coo = nullptr;
    if (!o.mtx.empty()) {
        std::printf("Loading MTX: %s\n", o.mtx.c_str());
        CHECK(vcsr_mtx_read(o.mtx.c_str(), o.expand ? 1 : 0, &coo));
    } else {
        std::printf("Generating: cfg%d seed=%llu\n", o.gen, o.seed);
        CHECK(vcsr_gen_coo(o.gen, (uint64_t)o.seed, &coo));
    }
    vcsr_csr* csr = nullptr;
    CHECK(vcsr_coo_to_csr(coo, &csr));
    vcsr_coo_free(coo);
    vcsr_csr_view A;
    CHECK(vcsr_csr_view_get(csr, &A));
    std::printf("Matrix: %d x %d, nnz=%d\n", A.M, A.N, A.nnz);
    std::printf("Params: O=%d, segw=%d, bundle=%d, tileK=%d, repeat=%d\n", o.O, o.segw, o.bundle,
                o.tileK, o.repeat);

    const int32_t O = o.O;
    std::vector<float> hB((size_t)A.N * O);
    CHECK(vcsr_gen_dense((uint64_t)o.seed + 1, o.gen == 5 ? 1 : 0, A.N, O, hB.data()));
    const double flop = 2.0 * (double)A.nnz * O;
    const double bytes_alg = 4.0 * (A.M + 1) + 8.0 * A.nnz + 4.0 * A.N * O + 4.0 * (double)A.M * O;
    auto gflops = [&](double ms) { return flop / (ms * 1e6); };

    std::vector<float> ref;  // CPU result, computed on demand
    std::vector<double> row_l1;
    double bmax = 0;
    auto need_ref = [&] {
        if (!ref.empty() || A.M == 0) return;
        ref.resize((size_t)A.M * O);
        CHECK(spmm_csr_cpu(A.M, A.row_ptr, A.col, A.val, hB.data(), O, ref.data(), o.threads));
        row_l1.assign((size_t)A.M, 0.0);
        for (int32_t r = 0; r < A.M; ++r)
            for (int32_t p = A.row_ptr[r]; p < A.row_ptr[r + 1]; ++p)
                row_l1[(size_t)r] += std::fabs((double)A.val[p]);
        for (float x : hB) bmax = std::max(bmax, (double)std::fabs(x));
    };

    const bool want_gpu = all || o.algo != "cpu";
    int32_t ndev = 0;
    vcsr_device_count(&ndev);
    if (want_gpu && ndev <= 0) {
        std::fprintf(stderr, "spmm_vcsr: no GPU visible; GPU algorithms need one\n");
        return 2;
    }
    void* st = nullptr;
    float *dB = nullptr, *dC = nullptr, *dval = nullptr;
    int32_t *drp = nullptr, *dcol = nullptr;
    const size_t bytesB = (size_t)A.N * O * sizeof(float), bytesC = (size_t)A.M * O * sizeof(float);
    if (want_gpu) {
        char name[128];
        CHECK(vcsr_device_name(name, sizeof(name)));
        std::printf("Device: %s\n", name);
        CHECK(vcsr_stream_create(&st));
        CHECK(vcsr_dev_malloc((void**)&dB, bytesB));
        CHECK(vcsr_dev_malloc((void**)&dC, bytesC));
        CHECK(vcsr_dev_malloc((void**)&drp, sizeof(int32_t) * ((size_t)A.M + 1)));
        CHECK(vcsr_dev_malloc((void**)&dcol, sizeof(int32_t) * (size_t)A.nnz));
        CHECK(vcsr_dev_malloc((void**)&dval, sizeof(float) * (size_t)A.nnz));
        CHECK(vcsr_memcpy_h2d(dB, hB.data(), bytesB, st));
        CHECK(vcsr_memcpy_h2d(drp, A.row_ptr, sizeof(int32_t) * ((size_t)A.M + 1), st));
        CHECK(vcsr_memcpy_h2d(dcol, A.col, sizeof(int32_t) * (size_t)A.nnz, st));
        CHECK(vcsr_memcpy_h2d(dval, A.val, sizeof(float) * (size_t)A.nnz, st));
    }

    auto report_check = [&](const char* name) {
        if (!o.check) return;
        need_ref();
        std::vector<float> hC((size_t)A.M * O);
        CHECK(vcsr_memcpy_d2h(hC.data(), dC, bytesC, st));
        Check c = compare(hC, ref, row_l1, bmax, O);
        std::printf("L2 diff (%s vs CPU CSR): rel=%.3e max_abs=%.3e max_abs/tol=%.3f %s\n", name,
                    c.rel_l2, c.max_abs, c.max_ratio, c.ok ? "PASS" : "FAIL");
    };
    auto report_roofline = [&](double ms) {
        const double gbs = bytes_alg / (ms * 1e-3) / 1e9;
        std::printf("roofline: bytes_alg=%.1f MB  %.1f GB/s  %.2f%% of 8000 GB/s\n",
                    bytes_alg / 1e6, gbs, 100.0 * gbs / 8000.0);
    };

    std::printf("\n");
    if (all || o.algo == "cpu") {
        need_ref();
        std::vector<float> tmp((size_t)A.M * O);
        double best = 1e300, sum = 0;
        for (int it = 0; it < std::max(1, std::min(o.repeat, 3)); ++it) {
            const double t0 = now_ms();
            CHECK(spmm_csr_cpu(A.M, A.row_ptr, A.col, A.val, hB.data(), O, tmp.data(), o.threads));
            const double t = now_ms() - t0;
            best = std::min(best, t);
            sum += t;
        }
        std::printf("%-12s%8.3f ms %9.2f GFLOP/s  [threads=%d]\n", "CPU (csr):", best, gflops(best),
                    o.threads);
    }
    if (all || o.algo == "rocsparse") {
        // The vendor library, set up and torn down on every call with only
        // the SpMM timed, as the reference's cuSPARSE wrapper does.
        float ms = 0, sum = 0;
        for (int it = 0; it < o.warmup; ++it)
            CHECK(spmm_csr_vendor(A.M, A.N, A.nnz, drp, dcol, dval, dB, O, dC, st, &ms));
        for (int it = 0; it < o.repeat; ++it) {
            CHECK(vcsr_memset_d(dC, 0, bytesC, st));
            CHECK(spmm_csr_vendor(A.M, A.N, A.nnz, drp, dcol, dval, dB, O, dC, st, &ms));
            sum += ms;
        }
        report_check("rocsparse");
        report_roofline(sum / o.repeat);
        std::printf("%-12s%8.3f ms %9.2f GFLOP/s  (vendor)\n", "rocSPARSE:", sum / o.repeat,
                    gflops(sum / o.repeat));
    }
    if (all || o.algo == "aspt") {
        float ms = 0, sum = 0;
        for (int it = 0; it < o.warmup; ++it)
            CHECK(spmm_csr_wave(A.M, A.N, drp, dcol, dval, dB, O, dC, st, &ms));
        for (int it = 0; it < o.repeat; ++it) {
            CHECK(vcsr_memset_d(dC, 0, bytesC, st));
            CHECK(spmm_csr_wave(A.M, A.N, drp, dcol, dval, dB, O, dC, st, &ms));
            sum += ms;
        }
        report_check("aspt");
        report_roofline(sum / o.repeat);
        std::printf("%-12s%8.3f ms %9.2f GFLOP/s\n", "ASpT (wave):", sum / o.repeat,
                    gflops(sum / o.repeat));
    }
    if (all || o.algo == "csr") {
        float ms = 0, sum = 0;
        for (int it = 0; it < o.warmup; ++it)
            CHECK(spmm_csr_naive(A.M, drp, dcol, dval, dB, O, dC, st, &ms));
        for (int it = 0; it < o.repeat; ++it) {
            CHECK(vcsr_memset_d(dC, 0, bytesC, st));
            CHECK(spmm_csr_naive(A.M, drp, dcol, dval, dB, O, dC, st, &ms));
            sum += ms;
        }
        report_check("csr");
        report_roofline(sum / o.repeat);
        std::printf("%-12s%8.3f ms %9.2f GFLOP/s\n", "CSR (naive):", sum / o.repeat,
                    gflops(sum / o.repeat));
    }
    // kind: 0 = spmm_vcsr (tile kernel), 1 = spmm_vcsr_mfma (group dense
    // tiles), 2 = spmm_vcsr on fixed 16-row windows (FastSpMM's layout).
    auto run_vcsr = [&](const char* label, int lay, int segw, int bundle, int kind) {
        const bool mfma = kind == 1;
        vcsr_fmt* fmt = nullptr;
        const double t0 = now_ms();
        const bool from_file = kind == 0 && !o.load_fmt.empty();
        if (from_file) {
            CHECK(vcsr_fmt_load(o.load_fmt.c_str(), &fmt));
            vcsr_arrays la;
            CHECK(vcsr_fmt_arrays(fmt, &la));
            if (la.M != A.M || la.N != A.N) {
                std::fprintf(stderr, "spmm_vcsr: %s holds a %d x %d format, the matrix is %d x %d\n",
                             o.load_fmt.c_str(), la.M, la.N, A.M, A.N);
                std::exit(1);
            }
            std::printf("format: loaded from %s\n", o.load_fmt.c_str());
        } else {
            CHECK(vcsr_build(csr, segw, bundle, lay, o.threads, &fmt));
        }
        if (kind == 0 && !o.save_fmt.empty()) {
            CHECK(vcsr_fmt_save(fmt, o.save_fmt.c_str()));
            std::printf("format: saved to %s\n", o.save_fmt.c_str());
        }
        if (kind == 2) {
            CHECK(vcsr_fmt_set_tile_rows(fmt, 16));
            CHECK(vcsr_fmt_set_tile_windows(fmt, 1));
        }
        const double tb = now_ms() - t0;
        vcsr_arrays v;
        CHECK(vcsr_fmt_arrays(fmt, &v));
        const double t1 = now_ms();
        CHECK(vcsr_fmt_upload(fmt, st));
        const double tu = now_ms() - t1;
        std::printf("format: layout=%s segw=%d bundle=%d groups=%d slots=%lld (%.2fx nnz) "
                    "build=%.1f ms upload=%.1f ms\n",
                    v.layout == VCSR_LAYOUT_H ? "H" : (v.layout == VCSR_LAYOUT_S ? "S" : "TC"),
                    v.segw, v.bundle, v.num_groups, (long long)v.num_slots,
                    A.nnz ? (double)v.num_slots / A.nnz : 0.0, tb, tu);
        float ms = 0, sum = 0;
        auto once = [&] {
            CHECK(vcsr_memset_d(dC, 0, bytesC, st));
            if (mfma) CHECK(spmm_vcsr_mfma(fmt, dB, O, dC, st, &ms));
            else CHECK(spmm_vcsr(fmt, dB, O, o.tileK, dC, st, &ms));
        };
        for (int it = 0; it < o.warmup; ++it) once();
        for (int it = 0; it < o.repeat; ++it) {
            once();
            sum += ms;
        }
        report_check(label);
        report_roofline(sum / o.repeat);
        // Utilisation of the matrix cores, for the MFMA kernel and for the
        // default kernel when its view has 16-row (MFMA) tiles: useful FLOPs
        // over issued MFMA FLOPs (padding of the dense tiles), and the issued
        // rate over the dense FP32 MFMA peak of MI355X (157.3 TFLOP/s).
        int64_t ops = 0;
        int32_t fpo = 0;
        if (mfma) CHECK(vcsr_mfma_work(fmt, O, 0, &ops, &fpo));
        else CHECK(vcsr_tile_mfma_work(fmt, O, &ops, &fpo));
        if (ops > 0) {
            const double issued = (double)ops * fpo;
            const double rate = issued / ((sum / o.repeat) * 1e-3) / 1e12;
            std::printf("mfma: %lld instructions, %.3f GFLOP issued, useful %.1f%%, "
                        "%.2f TFLOP/s issued = %.2f%% of 157.3 TFLOP/s FP32 MFMA peak\n",
                        (long long)ops, issued / 1e9,
                        issued > 0 ? 100.0 * 2.0 * A.nnz * O / issued : 0.0, rate,
                        100.0 * rate / 157.3);
        }
        std::printf("%-12s%8.3f ms %9.2f GFLOP/s  [segw=%d,bundle=%d,tileK=%d,groups=%d]\n", label,
                    sum / o.repeat, gflops(sum / o.repeat), v.segw, v.bundle, o.tileK,
                    v.num_groups);
        vcsr_fmt_free(fmt);
    };
    if (all || o.algo == "vcsr") run_vcsr("VCSR (seg):", layout, o.segw, o.bundle, 0);
    if (all || o.algo == "vcsr_mfma") run_vcsr("VCSR-MFMA:", layout, o.segw, o.bundle, 1);
    if (all || o.algo == "vcsr_tc") run_vcsr("VCSR-TC:", VCSR_LAYOUT_TC, 16, 16, 1);
    if (all || o.algo == "fast") run_vcsr("FastSpMM:", layout, o.segw, o.bundle, 2);

    if (want_gpu) {
        vcsr_dev_free(dB);
        vcsr_dev_free(dC);
        vcsr_dev_free(drp);
        vcsr_dev_free(dcol);
        vcsr_dev_free(dval);
        vcsr_stream_destroy(st);
    }
    vcsr_csr_free(csr);
    return 0;
}
