/* cujev_gemm_tune: builds the tuned hipBLASLt algorithm table for the
 * hipBLASLt this program links (the one a torch-free process loads, e.g. an
 * engine driven by the reference's ctypes layer or a C caller).
 *
 *   cujev_gemm_tune OUT_DIR M:K[,M:K...] N[,N...]
 *
 * writes OUT_DIR/gemm_table_gfx950_hipblaslt<version>.txt with one line
 * "N M K f32out index" per shape, each the fastest of all hipBLASLt solutions
 * that support it (timed on random bf16 buffers). */
#include "kernels/kernels.h"

#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

static std::vector<int> parse_ints(const char *s, char sep) {
    std::vector<int> v;
    while (*s) {
        v.push_back(atoi(s));
        const char *c = strchr(s, sep);
        if (!c)
            break;
        s = c + 1;
    }
    return v;
}

__global__ void fill_kernel(bf16_t *p, size_t n, unsigned seed, float scale) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        unsigned x = (unsigned)i * 2654435761u ^ seed;
        x ^= x >> 15;
        x *= 2246822519u;
        x ^= x >> 13;
        const float u = ((x & 0xffffff) / 16777216.0f - 0.5f) * scale;
        p[i] = (bf16_t)u;
    }
}

int main(int argc, char **argv) {
    if (argc != 4) {
        fprintf(stderr, "usage: %s OUT_DIR M:K[,M:K...] N[,N...]\n", argv[0]);
        return 2;
    }
    std::vector<std::pair<int, int>> shapes;
    for (const char *s = argv[2]; *s;) {
        int M = 0, K = 0;
        if (sscanf(s, "%d:%d", &M, &K) != 2 || M <= 0 || K <= 0) {
            fprintf(stderr, "bad shape list %s\n", argv[2]);
            return 2;
        }
        shapes.push_back({M, K});
        const char *c = strchr(s, ',');
        if (!c)
            break;
        s = c + 1;
    }
    const std::vector<int> tokens = parse_ints(argv[3], ',');
    size_t maxX = 0, maxW = 0, maxY = 0;
    for (auto &sh : shapes)
        for (int N : tokens) {
            maxX = std::max(maxX, (size_t)N * sh.second);
            maxW = std::max(maxW, (size_t)sh.first * sh.second);
            maxY = std::max(maxY, (size_t)N * sh.first);
        }
    const size_t WS = 64 << 20;
    bf16_t *X, *W, *Y;
    void *ws;
    if (hipMalloc(&X, maxX * 2) != hipSuccess || hipMalloc(&W, maxW * 2) != hipSuccess ||
        hipMalloc(&Y, maxY * 2) != hipSuccess || hipMalloc(&ws, WS) != hipSuccess) {
        fprintf(stderr, "hipMalloc failed\n");
        return 1;
    }
    hipLaunchKernelGGL(fill_kernel, dim3(1024), dim3(256), 0, 0, X, maxX, 1u, 2.0f);
    hipLaunchKernelGGL(fill_kernel, dim3(1024), dim3(256), 0, 0, W, maxW, 2u, 0.05f);
    hipStream_t stream;
    if (hipStreamCreate(&stream) != hipSuccess || hipGetLastError() != hipSuccess) {
        fprintf(stderr, "stream creation or the operand fill failed\n");
        return 1;
    }
    cujev_gemm *g;
    if (cujev_gemm_create(&g, ws, WS) != 0) {
        fprintf(stderr, "hipblasLtCreate failed\n");
        return 1;
    }
    const int ver = cujev_gemm_version(g);
    std::string path = std::string(argv[1]) + "/gemm_table_gfx950_hipblaslt" + std::to_string(ver) +
                       ".txt";
    std::string body = "# hipblaslt " + std::to_string(ver) + "\n# shapes " + argv[2] +
                       ", tokens " + argv[3] + "; columns: N M K f32out index\n";
    for (auto &sh : shapes)
        for (int N : tokens) {
            int idx = -1;
            float best = 0.f, heur = 0.f;
            if (cujev_gemm_tune(g, X, W, Y, 0, N, sh.first, sh.second, stream, &idx, &best,
                                &heur) != 0) {
                fprintf(stderr, "N=%d M=%d K=%d: no solution ran\n", N, sh.first, sh.second);
                return 1;
            }
            printf("N=%5d M=%6d K=%5d: heuristic %7.1f us -> %7.1f us (x%.2f, solution %d)\n", N,
                   sh.first, sh.second, heur, best, heur / best, idx);
            fflush(stdout);
            body += std::to_string(N) + " " + std::to_string(sh.first) + " " +
                    std::to_string(sh.second) + " 0 " + std::to_string(idx) + "\n";
        }
    FILE *f = fopen(path.c_str(), "w");
    if (!f || fputs(body.c_str(), f) < 0) {
        fprintf(stderr, "cannot write %s\n", path.c_str());
        return 1;
    }
    fclose(f);
    printf("wrote %s\n", path.c_str());
    cujev_gemm_destroy(g);
    return 0;
}
