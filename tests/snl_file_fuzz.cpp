// Driver for the `.snl` reader under the address and undefined-behaviour sanitizers (test
// infrastructure, CPU only; built and run by tests/test_snl_file_fuzz.py).  For every file named on
// the command line it runs snl::SnlFile::open and SnlFile::config, and for each tensor the reader
// accepted it checks, in 128-bit arithmetic, that the tensor's quants and scales lie inside the
// file, then reads their first and last bytes.  One line per file: "<i> ok", or "<i> rejected: <why>";
// a tensor placed past the end prints "<i> bounds <name>" and the exit status is 1.
#include <sys/stat.h>

#include <cstdio>
#include <string>

#include "snl_file.h"

int main(int argc, char** argv) {
    static const char* const kNames[] = {"embed", "norm", "l0.down", "lm_head", "l0.gate_up"};
    volatile unsigned sink = 0;
    int status = 0;
    for (int i = 1; i < argc; ++i) {
        snl::SnlFile f;
        std::string err;
        snl::FileConfig c;
        if (!f.open(argv[i], &err) || !f.config(&c, &err)) {
            printf("%d rejected: %s\n", i, err.c_str());
            continue;
        }
        struct stat st;
        if (stat(argv[i], &st) != 0) return 2;
        const unsigned __int128 size = (unsigned __int128)st.st_size;
        for (const char* name : kNames) {
            const snl::FileTensor* t = f.find(name);
            if (!t) continue;
            unsigned __int128 n = 1;
            for (int64_t d : t->shape) n *= (unsigned __int128)d;
            const unsigned __int128 qb = t->dtype == snl::FD_F32 ? n * 4 : t->dtype == snl::FD_Q8_0 ? n : n / 2;
            const unsigned __int128 sb = t->dtype == snl::FD_F32 ? 0 : n / 32 * 4;
            if (qb != t->quant_bytes() || sb != t->scale_bytes() || t->offset + qb > size ||
                t->scales_offset + sb > size) {
                printf("%d bounds %s\n", i, name);
                status = 1;
                continue;
            }
            if (qb) sink += f.quants(*t)[0] + f.quants(*t)[(size_t)qb - 1];
            if (sb) sink += f.scales(*t)[0] + f.scales(*t)[(size_t)sb - 1];
        }
        printf("%d ok\n", i);
    }
    return status;
}
