// Shared helpers of the per-task drivers: argument parsing, flat-binary file
// reads, and the reference's error behaviour (print, exit(1)) on top of the
// library's status codes.  Host-only C++; everything on the GPU goes through
// the C ABI in vdttfs.h.
#pragma once

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <map>
#include <string>
#include <vector>

#include "vdttfs.h"

#define VD_CHECK(call)                                                                      \
    do {                                                                                    \
        const int vd_rc_ = (call);                                                          \
        if (vd_rc_ != VDTTFS_OK) {                                                          \
            std::cerr << "vdttfs error " << vd_rc_ << " at " << __FILE__ << ":" << __LINE__ \
                      << ": " << vdttfs_last_error() << std::endl;                          \
            std::exit(1);                                                                   \
        }                                                                                   \
    } while (0)

// --key value pairs; a key given without a value reads as "1".
class Args {
  public:
    Args(int argc, char** argv) {
        for (int i = 1; i < argc; ++i) {
            std::string k = argv[i];
            if (k.rfind("--", 0) != 0) {
                std::cerr << "unexpected argument " << k << std::endl;
                std::exit(2);
            }
            k = k.substr(2);
            if (i + 1 < argc && std::string(argv[i + 1]).rfind("--", 0) != 0)
                kv_[k] = argv[++i];
            else
                kv_[k] = "1";
        }
    }
    std::string s(const std::string& k, const std::string& d) const {
        auto it = kv_.find(k);
        return it == kv_.end() ? d : it->second;
    }
    int i(const std::string& k, int d) const { return std::stoi(s(k, std::to_string(d))); }
    float f(const std::string& k, float d) const {
        auto it = kv_.find(k);
        return it == kv_.end() ? d : std::stof(it->second);
    }

  private:
    std::map<std::string, std::string> kv_;
};

// Reads exactly n floats / ints from `path` at byte offset `off`; exits as the
// reference's loaders do when the file is missing (and also when it is short).
template <class T>
inline void read_exact(const std::string& path, T* dst, size_t n, size_t off = 0) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) {
        std::cerr << "Cannot open " << path << std::endl;
        std::exit(1);
    }
    f.seekg((std::streamoff)off, std::ios::beg);
    f.read(reinterpret_cast<char*>(dst), (std::streamsize)(n * sizeof(T)));
    if ((size_t)f.gcount() != n * sizeof(T)) {
        std::cerr << "Short read from " << path << " (" << f.gcount() << " of " << n * sizeof(T)
                  << " bytes)" << std::endl;
        std::exit(1);
    }
}

// One-hot row -> class: the last entry > 0.5, as the loops of T1V:314 /
// T2V:392 leave it; -1 if none.
inline int onehot_class(const float* row, int c) {
    int t = -1;
    for (int i = 0; i < c; ++i)
        if (row[i] > 0.5f) t = i;
    return t;
}

inline double seconds_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

// Device buffer owned by a driver (freed at scope exit).
struct DevBuf {
    vdttfs_ctx* ctx = nullptr;
    void* p = nullptr;
    DevBuf(vdttfs_ctx* c, size_t bytes) : ctx(c) { VD_CHECK(vdttfs_dev_alloc(ctx, bytes, &p)); }
    ~DevBuf() {
        if (p) vdttfs_dev_free(ctx, p);
    }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    template <class T>
    T* as() const {
        return static_cast<T*>(p);
    }
};
