// st_host.h - the host side of the fmt=6 container reader (st_host.cpp): the safetensors
// shard index with the header rules of c/st.h:241-331, and the reads.  No device code: the
// CPU test suite also builds st_host.cpp alone under AddressSanitizer.
#pragma once

#include <stdint.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#ifndef COLI_API
#define COLI_API extern "C" __attribute__((visibility("default")))
#endif

namespace coli {

// dtype codes (c/st.h:62-69 numbers BF16 0, F16 1, F32 2, U8/I8 3)
enum { kBF16 = 0, kF16 = 1, kF32 = 2, kU8 = 3 };
constexpr uint64_t kMaxHeader = 512ull << 20;
constexpr int kMaxDims = 8;

struct StTensor {
    int fd;
    int64_t off, nbytes, numel;
    int dtype, ndim;
    int64_t shape[kMaxDims];
};

// every shard of a container: its descriptors and the name index
struct Shards {
    std::vector<int> fds;
    std::vector<std::string> paths;
    std::unordered_map<std::string, StTensor> map;
    ~Shards() {
        for (int fd : fds) close(fd);
    }
};

// c/st.h:171-195: full pread in chunks of at most 1 GiB, EINTR retried, short reads named
bool pread_full(int fd, void *buf, int64_t n, int64_t off);
// c/st.h:241-331: one shard's header into the index; false (with a message) on a bad shard
bool index_shard(Shards &S, const std::string &path);
const StTensor *find(const Shards &S, const std::string &name);
// the tensor's bytes as f32 into out[numel] (c/st.h:399-428): F32, BF16 or F16
bool read_f32(const StTensor &t, float *out);

}  // namespace coli

// The opaque handle of coli_hip_st_* (include/coli_hip.h).
struct ColiHipSt {
    coli::Shards s;
    std::string dir;
};
