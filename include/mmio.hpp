// mmio.hpp -- Matrix Market coordinate input of the drop-in surface.
//
// Same struct and function as MuuSeoTia/VCSR_MC include/mmio.hpp:12-75 (COO, and
// read_matrix_market_coo with its banner, value and symmetry rules and its error texts), so the
// reference's driver compiles against this header unchanged.  Accepted input:
//   banner    "%%MatrixMarket matrix coordinate <field> <symmetry>", field real | integer |
//             pattern, symmetry general | symmetric | skew-symmetric (square only);
//   then      lines that are blank or start with '%' (after spaces, tabs and CRs) are skipped;
//             "M N count" (1 <= M, N < 2^31 - 1, 0 <= count <= 2^31 - 1);
//             count entries "row col [value]", one-based; pattern entries are 1.0, a value must
//             be a finite float; a symmetric entry off the diagonal also gives its mirror (skew:
//             with the sign flipped, and a skew diagonal must be zero); nothing may follow.
// Numbers are read with the grammar of a C++ stream extraction in the "C" locale (integers:
// optional sign and decimal digits; reals: optional sign, digits with one '.', an exponent only
// after a digit), so the reference's inputs and error texts carry over.
#pragma once
#include <algorithm>
#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

struct COO {
    int M{0}, N{0};
    std::vector<int> rows, cols;
    std::vector<float> vals;
};

namespace vcsrmc_mtx {

inline bool is_space(char ch) {
    return ch == ' ' || ch == '\t' || ch == '\n' || ch == '\v' || ch == '\f' || ch == '\r';
}

// A cursor over one line, read the way operator>> reads it.
class Fields {
public:
    explicit Fields(const std::string& s) : p_(s.data()), e_(s.data() + s.size()) {}

    bool word(std::string& out) {
        skip();
        const char* b = p_;
        while (p_ < e_ && !is_space(*p_)) ++p_;
        out.assign(b, p_);
        return p_ > b;
    }
    // Optional sign and decimal digits; fails on no digits or on overflow.
    bool integer(long long& out) {
        skip();
        const char* b = p_;
        if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
        const char* d = p_;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ == d) return false;
        const std::string text(b, p_);
        errno = 0;
        char* end = nullptr;
        out = std::strtoll(text.c_str(), &end, 10);
        return errno != ERANGE;
    }
    // Mantissa of digits with at most one '.', then an exponent only after a mantissa digit;
    // the collected characters must form a whole number that is finite as a double.
    bool real(double& out) {
        skip();
        std::string t;
        if (p_ < e_ && (*p_ == '+' || *p_ == '-')) t += *p_++;
        bool digit = false, dot = false, expo = false;
        while (p_ < e_) {
            const char ch = *p_;
            if (ch >= '0' && ch <= '9') {
                digit = true;
            } else if (ch == '.' && !dot && !expo) {
                dot = true;
            } else if ((ch == 'e' || ch == 'E') && !expo && digit) {
                expo = true;
                t += ch;
                ++p_;
                if (p_ < e_ && (*p_ == '+' || *p_ == '-')) t += *p_++;
                continue;
            } else {
                break;
            }
            t += ch;
            ++p_;
        }
        char* end = nullptr;
        out = std::strtod(t.c_str(), &end);
        if (t.empty() || end != t.c_str() + t.size()) return false;
        return std::fabs(out) != std::numeric_limits<double>::infinity();
    }
    bool more() {
        skip();
        return p_ < e_;
    }

private:
    void skip() {
        while (p_ < e_ && is_space(*p_)) ++p_;
    }
    const char* p_;
    const char* e_;
};

// Lines of a file (without the '\n'), read in large blocks.
class Lines {
public:
    explicit Lines(const std::string& path) : f_(std::fopen(path.c_str(), "rb")), buf_(1 << 20) {}
    ~Lines() {
        if (f_) std::fclose(f_);
    }
    Lines(const Lines&) = delete;
    Lines& operator=(const Lines&) = delete;
    bool ok() const { return f_ != nullptr; }

    bool next(std::string& line) {
        line.clear();
        bool any = false;
        for (;;) {
            if (pos_ == len_) {
                len_ = std::fread(buf_.data(), 1, buf_.size(), f_);
                pos_ = 0;
                if (len_ == 0) return any;
            }
            any = true;
            const char* b = buf_.data() + pos_;
            const char* nl = static_cast<const char*>(std::memchr(b, '\n', len_ - pos_));
            if (nl) {
                line.append(b, nl);
                pos_ += (size_t)(nl - b) + 1;
                return true;
            }
            line.append(b, len_ - pos_);
            pos_ = len_;
        }
    }
    // The next line holding data: not blank and not a '%' comment.
    bool next_data(std::string& line) {
        while (next(line)) {
            for (char ch : line) {
                if (ch == ' ' || ch == '\t' || ch == '\r') continue;
                if (ch != '%') return true;
                break;
            }
        }
        return false;
    }

private:
    std::FILE* f_;
    std::vector<char> buf_;
    size_t pos_ = 0, len_ = 0;
};

}  // namespace vcsrmc_mtx

inline COO read_matrix_market_coo(const std::string& path) {
    using vcsrmc_mtx::Fields;
    vcsrmc_mtx::Lines in(path);
    if (!in.ok()) throw std::runtime_error("Failed to open MTX: " + path);
    std::string line;
    if (!in.next(line)) throw std::runtime_error("Empty MTX file");
    std::string banner[5];
    {
        Fields f(line);
        for (std::string& w : banner)
            if (!f.word(w)) break;
    }
    const std::string& field = banner[3];
    const std::string& symmetry = banner[4];
    if (banner[0] != "%%MatrixMarket" || banner[1] != "matrix" || banner[2] != "coordinate")
        throw std::runtime_error("Expected a Matrix Market coordinate matrix");
    const bool pattern = field == "pattern";
    if (field != "real" && field != "integer" && !pattern)
        throw std::runtime_error("Unsupported MTX field: " + field);
    const bool general = symmetry == "general", skew = symmetry == "skew-symmetric";
    if (!general && symmetry != "symmetric" && !skew)
        throw std::runtime_error("Unsupported MTX symmetry: " + symmetry);

    if (!in.next_data(line)) throw std::runtime_error("Missing MTX dimensions");
    long long m = 0, n = 0, count = 0;
    {
        Fields f(line);
        const bool read = f.integer(m) && f.integer(n) && f.integer(count);
        if (!read || m <= 0 || n <= 0 || m >= INT_MAX || n >= INT_MAX || count < 0 ||
            count > INT_MAX)
            throw std::runtime_error("Invalid or unsupported MTX dimensions/nnz");
    }
    if (!general && m != n) throw std::runtime_error("Symmetric MTX must be square");

    COO coo;
    coo.M = (int)m;
    coo.N = (int)n;
    // (the declared count only sizes a first reservation: the file may hold fewer entries)
    const size_t room = std::min<size_t>((size_t)count * (general ? 1 : 2), (size_t)1 << 24);
    coo.rows.reserve(room);
    coo.cols.reserve(room);
    coo.vals.reserve(room);
    auto add = [&coo](long long r, long long c, float v) {
        if (coo.vals.size() >= (size_t)INT_MAX)
            throw std::runtime_error("Expanded MTX exceeds 32-bit nnz limit");
        coo.rows.push_back((int)r);
        coo.cols.push_back((int)c);
        coo.vals.push_back(v);
    };
    for (long long i = 0; i < count; ++i) {
        if (!in.next_data(line)) throw std::runtime_error("Truncated MTX data");
        Fields f(line);
        long long r = 0, c = 0;
        double v = 1.0;
        if (!f.integer(r) || !f.integer(c) || (!pattern && !f.real(v)))
            throw std::runtime_error("Bad MTX entry at index " + std::to_string(i));
        if (f.more()) throw std::runtime_error("Extra fields in MTX entry");
        if (r < 1 || r > m || c < 1 || c > n)
            throw std::runtime_error(
                "MTX row/column index out of range (expected one-based indices)");
        if (!std::isfinite(v) || std::fabs(v) > (double)std::numeric_limits<float>::max())
            throw std::runtime_error("MTX value is not finite FP32");
        if (skew && r == c && v != 0)
            throw std::runtime_error("Skew-symmetric MTX diagonal must be zero");
        add(r - 1, c - 1, (float)v);
        if (!general && r != c) add(c - 1, r - 1, (float)(skew ? -v : v));
    }
    if (in.next_data(line)) throw std::runtime_error("Extra entries after declared MTX nnz");
    return coo;
}
