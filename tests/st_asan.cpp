// Test driver for the container reader's host side (qwen3.c_amd/csrc/st_host.cpp) built
// alone under AddressSanitizer and UBSan by tests/test_container.py: for every directory
// named on the command line, coli_hip_st_open, then every indexed tensor looked up and read
// (raw bytes, and as f32 for the float dtypes; reads of more than 1 MiB are skipped), then
// coli_hip_st_close.  Prints one line per directory: "open" or "refused" and the tensor
// count.  Exit status 0 unless a sanitizer stops the run.
#include "../qwen3.c_amd/csrc/st_host.h"

#include <stdio.h>

#include <vector>

extern "C" ColiHipSt *coli_hip_st_open(const char *dir);
extern "C" void coli_hip_st_close(ColiHipSt *st);
extern "C" int coli_hip_st_find(const ColiHipSt *st, const char *name, int *dtype, int64_t *numel, int64_t *nbytes,
                                int *ndim, int64_t *shape);
extern "C" int64_t coli_hip_st_read_f32(const ColiHipSt *st, const char *name, float *out, int64_t cap);
extern "C" int64_t coli_hip_st_read_raw(const ColiHipSt *st, const char *name, void *out, int64_t cap);

int main(int argc, char **argv) {
    for (int a = 1; a < argc; a++) {
        ColiHipSt *st = coli_hip_st_open(argv[a]);
        if (!st) {
            printf("refused %s\n", argv[a]);
            continue;
        }
        int n = 0;
        for (const auto &kv : st->s.map) {
            int dt = -1, nd = 0;
            int64_t ne = 0, nb = 0, shape[8];
            if (!coli_hip_st_find(st, kv.first.c_str(), &dt, &ne, &nb, &nd, shape)) continue;
            n++;
            if (nb > (1 << 20)) continue;
            std::vector<unsigned char> raw((size_t)nb + 1);
            coli_hip_st_read_raw(st, kv.first.c_str(), raw.data(), nb);
            coli_hip_st_read_raw(st, kv.first.c_str(), raw.data(), nb > 0 ? nb - 1 : 0);   // a short cap: refused
            if (dt != 3) {
                std::vector<float> f((size_t)ne + 1);
                coli_hip_st_read_f32(st, kv.first.c_str(), f.data(), ne);
            }
        }
        printf("open %s %d\n", argv[a], n);
        coli_hip_st_close(st);
    }
    return 0;
}
