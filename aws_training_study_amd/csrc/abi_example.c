/*
 * A plain C caller of the C ABI (include/pcp_attention_hip.h): no Python,
 * no torch.  It is what a foreign-function binding of the history attention
 * does underneath — fill the parameter struct, put the tensors in device
 * memory, call the entry point on a stream, read the status — and the tests
 * run it against the Python path and the oracle.
 *
 *   abi_example check <params.bin>
 *       Prints the pcpa_check_params status of the pcpa_params struct stored
 *       in the file (no HIP call is made).
 *   abi_example run <dir> [calls]
 *       Reads params.bin, q.bin, kv.bin, table.bin and lens.bin from <dir>
 *       (raw little-endian arrays in the layouts the header describes),
 *       copies them to the GPU, calls pcpa_history_attention_lse once and
 *       writes out.bin (bf16) and lse.bin (float) to <dir>.  With `calls`,
 *       it then times that many back-to-back calls on the same stream and
 *       prints the host time per call and the device time per call.
 *
 * Built by aws_training_study_amd/build_native.py with gcc, linked against
 * the library and the HIP runtime.
 */
#define _POSIX_C_SOURCE 199309L /* clock_gettime */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "pcp_attention_hip.h"

static void* read_file(const char* dir, const char* name, size_t* size) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE* f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path);
        exit(2);
    }
    fseek(f, 0, SEEK_END);
    const long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    void* buf = malloc(n > 0 ? (size_t)n : 1);
    if (!buf || fread(buf, 1, (size_t)n, f) != (size_t)n) {
        fprintf(stderr, "cannot read %s\n", path);
        exit(2);
    }
    fclose(f);
    *size = (size_t)n;
    return buf;
}

static void write_file(const char* dir, const char* name, const void* data, size_t size) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE* f = fopen(path, "wb");
    if (!f || fwrite(data, 1, size, f) != size) {
        fprintf(stderr, "cannot write %s\n", path);
        exit(2);
    }
    fclose(f);
}

#define HIP_OK(call)                                                              \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess) {                                                   \
            fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(e_));           \
            exit(3);                                                              \
        }                                                                         \
    } while (0)

static void* to_device(const void* host, size_t size) {
    void* dev = NULL;
    HIP_OK(hipMalloc(&dev, size > 0 ? size : 1));
    if (size) HIP_OK(hipMemcpy(dev, host, size, hipMemcpyHostToDevice));
    return dev;
}

static double now_us(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec * 1e6 + t.tv_nsec * 1e-3;
}

static int check(const char* params_path) {
    FILE* f = fopen(params_path, "rb");
    pcpa_params p;
    if (!f || fread(&p, 1, sizeof p, f) != sizeof p) {
        fprintf(stderr, "cannot read %s\n", params_path);
        return 2;
    }
    fclose(f);
    const int32_t st = pcpa_check_params(&p);
    printf("status %d %s\n", (int)st, pcpa_status_string(st));
    return 0;
}

static int run(const char* dir, int calls) {
    size_t n_params, n_q, n_kv, n_table, n_lens;
    pcpa_params* p = (pcpa_params*)read_file(dir, "params.bin", &n_params);
    if (n_params != sizeof(pcpa_params)) {
        fprintf(stderr, "params.bin holds %zu bytes, pcpa_params is %zu\n", n_params, sizeof(pcpa_params));
        return 2;
    }
    const int32_t st = pcpa_check_params(p);
    if (st != PCPA_OK) {
        printf("status %d %s\n", (int)st, pcpa_status_string(st));
        return 1;
    }
    void* q = read_file(dir, "q.bin", &n_q);
    void* kv = read_file(dir, "kv.bin", &n_kv);
    void* table = read_file(dir, "table.bin", &n_table);
    void* lens = read_file(dir, "lens.bin", &n_lens);
    const size_t rows = (size_t)p->pcp_size * p->num_q_heads * p->local_q_len;
    const size_t kv_elem = p->kv_dtype == PCPA_DTYPE_BF16 ? 2 : 1;
    const size_t table_elem = (p->flags & PCPA_FLAG_TABLE_INT64) ? 8 : 4;
    const size_t blocks = (size_t)p->pcp_size * p->max_local_blocks;
    if (n_q != rows * p->head_dim * 2 ||
        n_kv != (size_t)p->num_pages * 2 * p->num_kv_heads * p->block_size * p->head_dim * kv_elem ||
        n_table != blocks * table_elem || n_lens != blocks * 4) {
        fprintf(stderr, "input sizes do not match params\n");
        return 2;
    }
    void* d_q = to_device(q, n_q);
    void* d_kv = to_device(kv, n_kv);
    void* d_table = to_device(table, n_table);
    void* d_lens = to_device(lens, n_lens);
    void* d_out = NULL;
    void* d_lse = NULL;
    HIP_OK(hipMalloc(&d_out, rows * p->head_dim * 2));
    HIP_OK(hipMalloc(&d_lse, rows * 4));
    hipStream_t stream;
    HIP_OK(hipStreamCreate(&stream));

    int32_t status = pcpa_history_attention_lse(p, d_q, d_kv, d_table, (const int32_t*)d_lens, d_out,
                                                (float*)d_lse, stream);
    if (status != PCPA_OK) {
        printf("status %d %s\n", (int)status, pcpa_status_string(status));
        return 1;
    }
    HIP_OK(hipStreamSynchronize(stream));
    void* out = malloc(rows * p->head_dim * 2);
    void* lse = malloc(rows * 4);
    HIP_OK(hipMemcpy(out, d_out, rows * p->head_dim * 2, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(lse, d_lse, rows * 4, hipMemcpyDeviceToHost));
    write_file(dir, "out.bin", out, rows * p->head_dim * 2);
    write_file(dir, "lse.bin", lse, rows * 4);
    printf("status 0 %s\n", pcpa_status_string(PCPA_OK));

    if (calls > 0) {
        hipEvent_t e0, e1;
        HIP_OK(hipEventCreate(&e0));
        HIP_OK(hipEventCreate(&e1));
        HIP_OK(hipEventRecord(e0, stream));
        const double t0 = now_us();
        for (int i = 0; i < calls; ++i) {
            status = pcpa_history_attention_lse(p, d_q, d_kv, d_table, (const int32_t*)d_lens, d_out,
                                                (float*)d_lse, stream);
            if (status != PCPA_OK) {
                printf("status %d %s\n", (int)status, pcpa_status_string(status));
                return 1;
            }
        }
        const double t_issue = now_us() - t0;
        HIP_OK(hipEventRecord(e1, stream));
        HIP_OK(hipEventSynchronize(e1));
        const double t_all = now_us() - t0;
        float device_ms = 0.f;
        HIP_OK(hipEventElapsedTime(&device_ms, e0, e1));
        printf("calls %d host_issue_us_per_call %.3f wall_us_per_call %.3f device_us_per_call %.3f\n", calls,
               t_issue / calls, t_all / calls, device_ms * 1e3 / calls);
        HIP_OK(hipEventDestroy(e0));
        HIP_OK(hipEventDestroy(e1));
    }
    HIP_OK(hipStreamDestroy(stream));
    hipFree(d_q);
    hipFree(d_kv);
    hipFree(d_table);
    hipFree(d_lens);
    hipFree(d_out);
    hipFree(d_lse);
    free(p);
    free(q);
    free(kv);
    free(table);
    free(lens);
    free(out);
    free(lse);
    return 0;
}

int main(int argc, char** argv) {
    if (argc >= 3 && strcmp(argv[1], "check") == 0) return check(argv[2]);
    if (argc >= 3 && strcmp(argv[1], "run") == 0) return run(argv[2], argc >= 4 ? atoi(argv[3]) : 0);
    fprintf(stderr, "usage: %s check <params.bin> | run <dir> [calls]\n", argv[0]);
    return 2;
}
