/*
 * q4rdna_c_check.c -- the C ABI used from plain C, the way a C/C++ host
 * (llama.cpp's ggml-cuda backend) would bind it: no Python, no torch.
 *
 * Builds a three-tensor sidecar image in memory, opens it on device 0, looks
 * weights up by ggml name and shape, and runs q4rdna_mul_mat, _add, _glu,
 * _batch and a two-GEMV plan against a double-precision CPU dot product of the same
 * tiles (IEEE fp16 scales).  Also checks the not-applicable paths leave the
 * output untouched.  Exit status 0 and "c abi ok" on success.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "q4rdna.h"

#define CHECK_HIP(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { \
    fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); return 1; } } while (0)
#define EXPECT(c) do { if (!(c)) { fprintf(stderr, "check failed at line %d: %s (%s)\n", __LINE__, #c, \
    q4rdna_last_error()); return 1; } } while (0)

static uint64_t lcg = 0x51EE0001u;
static uint32_t next_u32(void) { lcg = lcg * 6364136223846793005ull + 1442695040888963407ull; return (uint32_t)(lcg >> 32); }
static float next_gauss(void) {  /* sum of uniforms: enough for test data */
    float s = 0.0f;
    for (int i = 0; i < 12; ++i) s += (float)(next_u32() >> 8) / 16777216.0f;
    return s - 6.0f;
}

/* IEEE binary16 -> binary32, subnormals exact. */
static double half_to_double(uint16_t h) {
    int e = (h >> 10) & 31, m = h & 1023;
    double v = e == 0 ? ldexp(m, -24) : e == 31 ? (m ? NAN : INFINITY) : ldexp(1024 + m, e - 25);
    return (h & 0x8000) ? -v : v;
}
static uint16_t float_to_half_normal(float f) {  /* finite, normal-range test scales only */
    uint32_t b; memcpy(&b, &f, 4);
    uint32_t sign = (b >> 16) & 0x8000u, e = ((b >> 23) & 255u) - 127u + 15u, m = (b >> 13) & 1023u;
    return (uint16_t)(sign | (e << 10) | m);
}

/* Random tiles with sane scales: rows x cols weights. */
static void fill_tiles(uint8_t *t, uint32_t rows, uint32_t cols) {
    size_t n = (size_t)rows * cols * 34 / 64;
    for (size_t i = 0; i < n; ++i) t[i] = (uint8_t)next_u32();
    for (size_t tile = 0; tile < n / 1088; ++tile)
        for (int l = 0; l < 32; ++l) {
            float s = 0.002f + 0.02f * (float)(next_u32() >> 8) / 16777216.0f;
            uint16_t h = float_to_half_normal((next_u32() & 1) ? -s : s);
            memcpy(t + tile * 1088 + 2 * l, &h, 2);
        }
}

static int nibble(uint8_t b, int hi) { int v = hi ? (b >> 4) : (b & 15); return v >= 8 ? v - 16 : v; }

static void cpu_gemv(const uint8_t *t, uint32_t rows, uint32_t cols, const float *x, double *y, double *ay) {
    uint32_t groups = cols / 64;
    for (uint32_t r = 0; r < rows; ++r) {
        double s = 0, a = 0;
        for (uint32_t g = 0; g < groups; ++g) {
            const uint8_t *tile = t + ((size_t)(r / 32) * groups + g) * 1088;
            uint16_t h; memcpy(&h, tile + 2 * (r % 32), 2);
            double sc = half_to_double(h);
            for (int i = 0; i < 32; ++i) {
                uint8_t b = tile[64 + 32 * i + r % 32];
                double w0 = sc * nibble(b, 0), w1 = sc * nibble(b, 1);
                s += w0 * x[64 * g + 2 * i] + w1 * x[64 * g + 2 * i + 1];
                a += fabs(w0 * x[64 * g + 2 * i]) + fabs(w1 * x[64 * g + 2 * i + 1]);
            }
        }
        y[r] = s;
        if (ay) ay[r] = a;
    }
}

/* The per-row gate: |y - want| <= 1e-3 * max(|want|, 0.01 * rms(want)). */
static int gate_ok(const float *y, const double *want, uint32_t rows) {
    double ss = 0;
    for (uint32_t r = 0; r < rows; ++r) ss += want[r] * want[r];
    double floor_ = 0.01 * sqrt(ss / rows);
    for (uint32_t r = 0; r < rows; ++r) {
        double tol = 1e-3 * fmax(fabs(want[r]), floor_);
        if (!(fabs((double)y[r] - want[r]) <= tol)) {
            fprintf(stderr, "row %u: got %.9g want %.9g\n", r, y[r], want[r]);
            return 0;
        }
    }
    return 1;
}

static void put32(uint8_t *p, uint32_t v) { memcpy(p, &v, 4); }
static void put64(uint8_t *p, uint64_t v) { memcpy(p, &v, 8); }

int main(void) {
    const char *names[3] = {"blk.0.attn_q.weight", "blk.0.ffn_gate.weight", "blk.0.ffn_up.weight"};
    const uint32_t R[3] = {256, 512, 512}, C[3] = {1024, 512, 512};
    uint64_t data_offset = (48 + 96 * 3 + 4095) / 4096 * 4096, off[3], size[3], end = data_offset;
    for (int i = 0; i < 3; ++i) {
        off[i] = end;
        size[i] = (uint64_t)R[i] * C[i] * 34 / 64;
        end = (end + size[i] + 255) / 256 * 256;
    }
    uint8_t *img = calloc(end, 1);
    memcpy(img, "Q4RDNA1", 8);
    put32(img + 8, 1); put32(img + 12, 3); put32(img + 16, 64); put32(img + 20, 32); put32(img + 24, 1088);
    put32(img + 28, 0); put64(img + 32, data_offset); put64(img + 40, end - data_offset);
    for (int i = 0; i < 3; ++i) {
        uint8_t *e = img + 48 + 96 * i;
        strcpy((char *)e, names[i]);
        put32(e + 64, R[i]); put32(e + 68, C[i]); put64(e + 72, off[i]); put64(e + 80, size[i]); put64(e + 88, 0);
        fill_tiles(img + off[i], R[i], C[i]);
    }

    uint32_t count = 0;
    EXPECT(q4rdna_abi_version() == Q4RDNA_ABI_VERSION);
    EXPECT(q4rdna_sidecar_inspect(img, end, end, &count) == Q4RDNA_OK && count == 3);
    EXPECT(q4rdna_sidecar_inspect(img, end, end - 1, &count) < 0);  /* truncated file */
    q4rdna_sidecar *sc = NULL;
    EXPECT(q4rdna_sidecar_open_memory(img, end, 0, &sc) == Q4RDNA_OK);
    q4rdna_weight wq, wg, wu, tmp;
    EXPECT(q4rdna_find(sc, names[0], 1024, 256, &wq) == Q4RDNA_OK);        /* ne0 = K, ne1 = M */
    EXPECT(q4rdna_find(sc, names[0], 256, 1024, &tmp) == Q4RDNA_NOT_APPLICABLE);
    EXPECT(q4rdna_find(sc, "blk.0.attn_k.weight", 1024, 256, &tmp) == Q4RDNA_NOT_APPLICABLE);
    EXPECT(q4rdna_find(sc, names[1], 512, 512, &wg) == Q4RDNA_OK);
    EXPECT(q4rdna_find(sc, names[2], 512, 512, &wu) == Q4RDNA_OK);

    float *hx = malloc(1024 * sizeof(float)), *hy = malloc(512 * sizeof(float)), *hadd = malloc(512 * sizeof(float));
    double *want = malloc(512 * sizeof(double)), *want_g = malloc(512 * sizeof(double));
    for (int i = 0; i < 1024; ++i) hx[i] = next_gauss();
    for (int i = 0; i < 512; ++i) hadd[i] = next_gauss();
    float *dx, *dy, *dadd, *dy2;
    CHECK_HIP(hipMalloc((void **)&dx, 1024 * sizeof(float)));
    CHECK_HIP(hipMalloc((void **)&dy, 512 * sizeof(float)));
    CHECK_HIP(hipMalloc((void **)&dy2, 512 * sizeof(float)));
    CHECK_HIP(hipMalloc((void **)&dadd, 512 * sizeof(float)));
    CHECK_HIP(hipMemcpy(dx, hx, 1024 * sizeof(float), hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(dadd, hadd, 512 * sizeof(float), hipMemcpyHostToDevice));

    /* mul_mat */
    EXPECT(q4rdna_mul_mat(&wq, dx, 1024, dy, 256, NULL) == Q4RDNA_OK);
    CHECK_HIP(hipMemcpy(hy, dy, 256 * sizeof(float), hipMemcpyDeviceToHost));
    cpu_gemv(img + off[0], 256, 1024, hx, want, NULL);
    EXPECT(gate_ok(hy, want, 256));

    /* not applicable: wrong K leaves y untouched */
    CHECK_HIP(hipMemset(dy, 0x7f, 512 * sizeof(float)));
    EXPECT(q4rdna_mul_mat(&wq, dx, 512, dy, 256, NULL) == Q4RDNA_NOT_APPLICABLE);
    EXPECT(q4rdna_mul_mat(NULL, dx, 1024, dy, 256, NULL) == Q4RDNA_NOT_APPLICABLE);
    CHECK_HIP(hipMemcpy(hy, dy, 4, hipMemcpyDeviceToHost));
    uint32_t bits; memcpy(&bits, hy, 4);
    EXPECT(bits == 0x7f7f7f7fu);

    /* mul_mat_add */
    EXPECT(q4rdna_mul_mat_add(&wg, dx, 512, dadd, 512, dy, 512, NULL) == Q4RDNA_OK);
    CHECK_HIP(hipMemcpy(hy, dy, 512 * sizeof(float), hipMemcpyDeviceToHost));
    cpu_gemv(img + off[1], 512, 512, hx, want, NULL);
    for (int r = 0; r < 512; ++r) want[r] += hadd[r];
    EXPECT(gate_ok(hy, want, 512));

    /* mul_mat_glu: up * silu(gate) */
    EXPECT(q4rdna_mul_mat_glu(&wu, &wg, dx, 512, Q4RDNA_GLU_SWIGLU, dy, 512, NULL) == Q4RDNA_OK);
    EXPECT(q4rdna_mul_mat_glu(&wu, &wg, dx, 512, Q4RDNA_GLU_SWIGLU + 1, dy2, 512, NULL) == Q4RDNA_NOT_APPLICABLE);
    CHECK_HIP(hipMemcpy(hy, dy, 512 * sizeof(float), hipMemcpyDeviceToHost));
    cpu_gemv(img + off[2], 512, 512, hx, want, NULL);
    cpu_gemv(img + off[1], 512, 512, hx, want_g, NULL);
    for (int r = 0; r < 512; ++r) want[r] *= want_g[r] / (1.0 + exp(-want_g[r]));
    EXPECT(gate_ok(hy, want, 512));

    /* a two-GEMV plan */
    q4rdna_gemv_desc d[2];
    memset(d, 0, sizeof d);
    d[0].weight = wq; d[0].x = dx; d[0].y = dy;
    d[1].weight = wu; d[1].gate_tiles = wg.tiles; d[1].x = dx; d[1].y = dy2;
    q4rdna_plan *plan = NULL;
    EXPECT(q4rdna_plan_create(d, 2, 0, &plan) == Q4RDNA_OK);
    EXPECT(q4rdna_plan_workgroups(plan) >= 1);
    for (int rep = 0; rep < 2; ++rep) EXPECT(q4rdna_plan_launch(plan, NULL) == Q4RDNA_OK);
    CHECK_HIP(hipDeviceSynchronize());
    CHECK_HIP(hipMemcpy(hy, dy2, 512 * sizeof(float), hipMemcpyDeviceToHost));
    EXPECT(gate_ok(hy, want, 512));                       /* the SwiGLU result again */
    CHECK_HIP(hipMemcpy(hy, dy, 256 * sizeof(float), hipMemcpyDeviceToHost));
    cpu_gemv(img + off[0], 256, 1024, hx, want, NULL);
    EXPECT(gate_ok(hy, want, 256));
    q4rdna_plan_destroy(plan);

    /* mul_mat_batch: three vectors, x [3][1024], y [3][256] */
    {
        float *hxb = malloc(3 * 1024 * sizeof(float)), *hyb = malloc(3 * 256 * sizeof(float));
        for (int i = 0; i < 3 * 1024; ++i) hxb[i] = next_gauss();
        float *dxb, *dyb;
        CHECK_HIP(hipMalloc((void **)&dxb, 3 * 1024 * sizeof(float)));
        CHECK_HIP(hipMalloc((void **)&dyb, 3 * 256 * sizeof(float)));
        CHECK_HIP(hipMemcpy(dxb, hxb, 3 * 1024 * sizeof(float), hipMemcpyHostToDevice));
        EXPECT(q4rdna_mul_mat_batch(&wq, NULL, dxb, 3, NULL, dyb, NULL, NULL) == Q4RDNA_OK);
        EXPECT(q4rdna_mul_mat_batch(&wq, NULL, dxb, 9, NULL, dyb, NULL, NULL) == Q4RDNA_ERR_ARGUMENT);
        CHECK_HIP(hipMemcpy(hyb, dyb, 3 * 256 * sizeof(float), hipMemcpyDeviceToHost));
        for (int v = 0; v < 3; ++v) {
            cpu_gemv(img + off[0], 256, 1024, hxb + 1024 * v, want, NULL);
            EXPECT(gate_ok(hyb + 256 * v, want, 256));
        }
        CHECK_HIP(hipFree(dxb));
        CHECK_HIP(hipFree(dyb));
        free(hxb);
        free(hyb);
    }

    q4rdna_sidecar_close(sc);
    CHECK_HIP(hipFree(dx)); CHECK_HIP(hipFree(dy)); CHECK_HIP(hipFree(dy2)); CHECK_HIP(hipFree(dadd));
    free(img); free(hx); free(hy); free(hadd); free(want); free(want_g);
    printf("c abi ok\n");
    return 0;
}
