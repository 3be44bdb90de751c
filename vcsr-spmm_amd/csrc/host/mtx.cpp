// mtx.cpp - Matrix Market coordinate reader.
//
// Semantics follow read_matrix_market_coo (reference include/mmio.hpp:22-46):
//  * lines that are empty or start with '%' before the size line are skipped,
//    so the banner's `symmetric` / `pattern` qualifiers are ignored (:28-29);
//  * the first other line gives "M N nnz" (:30-31);
//  * then nnz whitespace-separated triples "r c v" are read, possibly across
//    line breaks (:36-37); a missing or malformed triple is an error (:37);
//  * indices are 1-based unless the FIRST entry has row 0 or column 0, in
//    which case all entries are taken as 0-based (:34,38-40);
//  * values are parsed as double and narrowed to float (:33,41);
//  * no size line at all is an error (:45).
// The file is read into memory once and tokenized with strtol/strtod-style
// scanning instead of iostreams.  On well-formed files the result is the
// same; the reference's undefined behaviour on a malformed size line becomes
// an error here.  expand_symmetric is an opt-in extension (off by default,
// as the reference never expands; SuiteSparse `cant` was run half-stored).
#include <cerrno>
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>

#include "core.hpp"

namespace vcsr {
namespace {

inline bool is_space(char ch) {
    return ch == ' ' || ch == '\t' || ch == '\n' || ch == '\r' || ch == '\v' ||
           ch == '\f';
}

// Extract a signed 32-bit integer like `istream >> int`: skip whitespace,
// optional sign, one or more digits; stops at the first non-digit.
bool scan_int(const char*& p, const char* end, int32_t& out) {
    while (p < end && is_space(*p)) ++p;
    const char* q = p;
    bool neg = false;
    if (q < end && (*q == '+' || *q == '-')) { neg = (*q == '-'); ++q; }
    if (q >= end || !std::isdigit((unsigned char)*q)) return false;
    int64_t v = 0;
    while (q < end && std::isdigit((unsigned char)*q)) {
        v = v * 10 + (*q - '0');
        if (v > (int64_t)INT32_MAX + 1) return false;
        ++q;
    }
    if (neg) v = -v;
    if (v < INT32_MIN || v > INT32_MAX) return false;
    out = (int32_t)v;
    p = q;
    return true;
}

// Extract a double: skip whitespace, then strtod on the token.
bool scan_double(const char*& p, const char* end, double& out) {
    while (p < end && is_space(*p)) ++p;
    if (p >= end) return false;
    // Copy the token so strtod never runs past `end`.
    char buf[128];
    size_t n = 0;
    while (p + n < end && !is_space(p[n]) && n < sizeof(buf) - 1) { buf[n] = p[n]; ++n; }
    buf[n] = '\0';
    char* stop = nullptr;
    errno = 0;
    double v = std::strtod(buf, &stop);
    if (stop == buf) return false;
    out = v;
    p += (stop - buf);
    return true;
}

bool banner_says(const std::string& banner, const char* word) {
    std::string low(banner);
    for (auto& ch : low) ch = (char)std::tolower((unsigned char)ch);
    std::istringstream iss(low);
    std::string tok;
    while (iss >> tok)
        if (tok == word) return true;
    return false;
}

}  // namespace

Coo read_mtx(const std::string& path, bool expand_symmetric) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw Error(2, "Failed to open MTX: " + path);
    std::string text((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    const char* p = text.data();
    const char* end = p + text.size();

    std::string banner;
    while (p < end) {
        const char* eol = (const char*)std::memchr(p, '\n', (size_t)(end - p));
        const char* line_end = eol ? eol : end;
        const char* next = eol ? eol + 1 : end;
        size_t len = (size_t)(line_end - p);
        if (len == 0) { p = next; continue; }
        if (p[0] == '%') {
            if (banner.empty() && len >= 2 && p[1] == '%') banner.assign(p, len);
            p = next;
            continue;
        }
        // Size line: "M N nnz" parsed from this line only (mmio.hpp:30-31).
        const char* h = p;
        int32_t M = 0, N = 0, nnz = 0;
        if (!scan_int(h, line_end, M) || !scan_int(h, line_end, N) ||
            !scan_int(h, line_end, nnz))
            throw Error(2, "Invalid MTX size line in " + path);
        if (M < 0 || N < 0 || nnz < 0) throw Error(2, "Negative MTX size in " + path);
        const bool symmetric = expand_symmetric && banner_says(banner, "symmetric");
        const bool skew = expand_symmetric && banner_says(banner, "skew-symmetric");
        Coo coo;
        coo.M = M;
        coo.N = N;
        size_t cap = (size_t)nnz * ((symmetric || skew) ? 2 : 1);
        coo.rows.reserve(cap);
        coo.cols.reserve(cap);
        coo.vals.reserve(cap);
        const char* q = next;
        bool one_based = true;
        for (int32_t i = 0; i < nnz; ++i) {
            int32_t r, c;
            double v;
            if (!scan_int(q, end, r) || !scan_int(q, end, c) || !scan_double(q, end, v))
                throw Error(2, "Bad MTX data in " + path);
            if (i == 0 && (r == 0 || c == 0)) one_based = false;
            const int32_t off = one_based ? 1 : 0;
            coo.rows.push_back(r - off);
            coo.cols.push_back(c - off);
            coo.vals.push_back((float)v);
            if ((symmetric || skew) && r != c) {
                coo.rows.push_back(c - off);
                coo.cols.push_back(r - off);
                coo.vals.push_back(skew ? -(float)v : (float)v);
            }
        }
        return coo;
    }
    throw Error(2, "Invalid MTX header or empty file: " + path);
}

}  // namespace vcsr
