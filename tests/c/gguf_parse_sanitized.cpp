// Host-only driver of the GGUF reader (qw6_amd/csrc/qw6_gguf.cpp) for a build
// under AddressSanitizer and UndefinedBehaviorSanitizer: opens every file of
// the directories given and, for each file the reader accepts, runs every
// query of include/qw6_gguf.h over every tensor index (and two past the end)
// and a set of keys. Built and run by tests/test_gguf_sanitized.py on the CPU;
// a sanitizer finding aborts the process. The two device-side functions the
// reader's upload paths call are replaced by failing stubs: no upload runs.
#include <dirent.h>
#include <stdio.h>

#include <string>
#include <vector>

#include "qw6_gguf.h"

namespace qw6 {
int qw6_fail(const char*, ...) { return -1; }
int ctx_device(const qw6_hip_ctx_t*) { return 0; }
}  // namespace qw6

extern "C" int qw6_hip_alloc(qw6_hip_ctx_t*, size_t, void**) { return -1; }
extern "C" int qw6_hip_experts_create(qw6_hip_ctx_t*, const qw6_hip_matrix_t*,
                                      const qw6_hip_matrix_t*, const qw6_hip_matrix_t*, uint32_t,
                                      qw6_hip_experts_t**) {
    return -1;
}

int main(int argc, char** argv) {
    unsigned opened = 0, rejected = 0;
    for (int a = 1; a < argc; a++) {
        DIR* d = opendir(argv[a]);
        if (!d) return 2;
        while (dirent* e = readdir(d)) {
            if (e->d_name[0] == '.') continue;
            const std::string path = std::string(argv[a]) + "/" + e->d_name;
            qw6_hip_gguf_t* g = nullptr;
            if (qw6_hip_gguf_open(path.c_str(), &g) != 0) {
                rejected++;
                continue;
            }
            opened++;
            uint32_t ver, nt, nkv, al;
            uint64_t doff, fsz;
            qw6_hip_gguf_header(g, &ver, &nt, &nkv, &al, &doff, &fsz);
            for (uint32_t i = 0; i < nt + 2; i++) {
                std::vector<char> name(128);   // the documented size, on the heap
                std::vector<int64_t> dims(4);
                uint32_t nd;
                int32_t ty;
                uint64_t off, span;
                if (qw6_hip_gguf_tensor(g, i, name.data(), &nd, dims.data(), &ty, &off, &span) == 0)
                    qw6_hip_gguf_find_tensor(g, name.data());
                const uint32_t counts[] = {0u, 1u, 2u, 3u, 256u, 0xffffffffu};
                for (uint32_t ne : counts) {
                    int32_t q;
                    uint32_t r, c;
                    uint64_t fo, eb;
                    qw6_hip_gguf_expert_pack(g, i, ne, &q, &r, &c, &fo, &eb);
                }
            }
            const char* keys[] = {"general.architecture", "general.alignment", "general.name",
                                  "qwen35moe.expert_count", "qwen35moe.block_count", "k", ""};
            for (const char* k : keys) {
                int64_t iv;
                double fv;
                qw6_hip_gguf_kv_type(g, k);
                qw6_hip_gguf_kv_int(g, k, &iv);
                qw6_hip_gguf_kv_float(g, k, &fv);
                // heap buffers of exactly cap bytes: a write past them is a finding
                const size_t caps[] = {1, 2, 7, 64};
                for (size_t cap : caps) {
                    std::vector<char> buf(cap);
                    qw6_hip_gguf_kv_str(g, k, buf.data(), cap);
                }
            }
            qw6_hip_gguf_close(g);
        }
        closedir(d);
    }
    printf("opened %u rejected %u\n", opened, rejected);
    return 0;
}
