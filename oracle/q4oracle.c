/*
 * q4oracle.c -- CPU oracle for the Q4_RDNA group-64 dequant-GEMV.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, the reference's
 * CPU algorithms for the hot path so that tests, the smoke check and the
 * bench's cpu_baseline leg can check the HIP library against them.  Nothing in
 * the product library links, loads or calls this code.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the reference root (source/...).
 *
 * Pinning status (what checks each function):
 *   q4o_fp16_to_f32            exhaustive vs a textbook IEEE binary16 decode (tests)
 *   q4o_fp16_to_f32_ref        exhaustive vs the textbook decode: equal except
 *                              subnormals, which it halves (the reference's bug)
 *   q4o_f32_to_fp16            vs numpy float16 RNE over finite floats; NaN quirk by case
 *   q4o_nibble_low/high        exhaustive 256-byte table vs closed form
 *   q4o_select_scale_sidecar   byte-identical to the compiled reference packer
 *                              (oracle/_ref) and to committed golden fixtures
 *   q4o_select_scale_experiment  byte-identical to the compiled reference CPU
 *                              experiment (oracle/_ref) and golden fixtures
 *   q4o_pack                   same as the scale selectors (tile placement)
 *   q4o_pack_mt                byte-identical to q4o_pack (tests)
 *   q4o_dequant                exhaustive closed form fp32(s)*q incl. signed zero
 *   q4o_gemv_seq_f32           vs fp64 brute force + planted-mistake checks
 *   q4o_gemv_seq_f32_mt        bit-identical to q4o_gemv_seq_f32 (tests)
 *   q4o_gemv_f64               vs numpy float64 matmul of the dequantized matrix
 *   q4o_silu                   vs long-double textbook g/(1+exp(-g)); the
 *                              reference's epilogue (llama.cpp unary.cuh) is not
 *                              vendored, so epilogue parity is "parity unpinned"
 *                              beyond the mathematics.
 *
 * Build: gcc -O2 -std=c11 -ffp-contract=off -fopenmp -fPIC -shared (no FMA
 * contraction, matching an x86-64 build of the reference without FMA
 * instructions; OpenMP only spreads independent rows over threads).  The
 * bench's CPU baseline also compiles it with -O3 -march=native on the host it
 * runs on; contraction stays off there too, so its results are the same bits.
 */
#include <fenv.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define Q4O_GROUP 64u
#define Q4O_TILE_ROWS 32u
#define Q4O_TILE_BYTES 1088u

/* ------------------------------------------------------------------ */
/* fp16 / bf16 conversions                                             */
/* ------------------------------------------------------------------ */

static float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* Exact IEEE binary16 -> binary32 from the definition of the format: a
 * subnormal is m * 2^-24, a normal number (1024 + m) * 2^(e - 25), e = 31 is
 * infinity or NaN.  This is what __half2float computes on the GPU
 * (source/q4rdna.cu:209,370,445): the decode of the runtime path. */
float q4o_fp16_to_f32(uint16_t h)
{
    const float sign = (h & 0x8000u) ? -1.0f : 1.0f;
    const int e = (h >> 10) & 31;
    const int m = h & 1023;
    if (e == 31) {
        if (m == 0) return sign * INFINITY;
        return bits_f32(((uint32_t)(h & 0x8000u) << 16) | 0x7fc00000u | ((uint32_t)m << 13));
    }
    if (e == 0) return sign * ldexpf((float)m, -24);
    return sign * ldexpf((float)(1024 + m), e - 25);
}

/* The reference CPU tools' binary16 decode, by its behaviour: exact for
 * zeros, normal numbers and infinities, but every subnormal comes out at half
 * its value (0x0001 gives 2^-25), because their normalisation loop uses the
 * exponent bias of a normal number.  The packers' scale search runs on this
 * decode, so the packed bytes depend on it: source/q4rdna_sidecar_pack.cpp:73-94,
 * source/q4rdna_cpu_experiment.cpp:39-60, and without the inf/NaN branch
 * source/q4rdna_gemv_bench.hip:163-187. */
float q4o_fp16_to_f32_ref(uint16_t h)
{
    const float exact = q4o_fp16_to_f32(h);
    const int subnormal = ((h >> 10) & 31) == 0 && (h & 1023) != 0;
    return subnormal ? 0.5f * exact : exact;
}

/* binary32 -> binary16 by the reference tools' behaviour: IEEE round to
 * nearest even (overflow to infinity, below half the smallest subnormal to a
 * signed zero), except that NaN becomes an infinity of the same sign
 * (source/q4rdna_sidecar_pack.cpp:96-124, q4rdna_cpu_experiment.cpp:62-100).
 * Computed from the value: |v| >= 65520 (halfway between 65504, the largest
 * finite half, and 2^16) is infinity; below 2^-14 the result is the number of
 * 2^-24 steps, rounded; otherwise 11 significant bits, rounded, where a round
 * up to 2048 carries into the exponent field by itself.  rintf rounds to
 * nearest even in the default rounding mode. */
uint16_t q4o_f32_to_fp16(float v)
{
    const uint16_t sign = signbit(v) ? 0x8000u : 0u;
    const float a = fabsf(v);
    if (isnan(v) || a >= 65520.0f) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x1p-14f) return (uint16_t)(sign | (uint16_t)rintf(a * 0x1p24f));
    int e;
    (void)frexpf(a, &e); /* a = f * 2^e, f in [0.5, 1): half exponent e - 1 */
    const uint32_t q = (uint32_t)rintf(ldexpf(a, 11 - e)); /* in [1024, 2048] */
    return (uint16_t)(sign | ((uint32_t)(e + 14) * 1024u + (q - 1024u)));
}

/* bf16 -> f32 (source/q4rdna_sidecar_pack.cpp:69-71). */
float q4o_bf16_to_f32(uint16_t v) { return bits_f32((uint32_t)v << 16); }

/* f32 -> bf16 round-to-nearest-even (fixture preparation only; finite input). */
uint16_t q4o_f32_to_bf16(float f)
{
    uint32_t b = f32_bits(f);
    uint32_t lsb = (b >> 16) & 1u;
    b += 0x7fffu + lsb;
    return (uint16_t)(b >> 16);
}

/* ------------------------------------------------------------------ */
/* signed nibble decode                                                */
/* ------------------------------------------------------------------ */

/* Two's-complement 4-bit codes: low nibble = even k, high nibble = odd k.
 * Restates source/q4rdna.cu:181-187 (same at source/q4rdna_gemv_bench.hip:50-56). */
int q4o_nibble_low(uint8_t b) { return (int)(int8_t)(uint8_t)(b << 4) >> 4; }
int q4o_nibble_high(uint8_t b) { return (int)(int8_t)b >> 4; }

/* ------------------------------------------------------------------ */
/* quantizers                                                          */
/* ------------------------------------------------------------------ */

/* int(t) for an integral float t, with the x86-64 cvttss2si result for values
 * outside int range (0x80000000).  The reference converts with int(...) on
 * x86-64, which yields INT_MIN there; clamping then gives -8. */
static int x86_float_to_int(float t)
{
    if (!(t >= -2147483648.0f && t < 2147483648.0f)) return (int)0x80000000u;
    return (int)t;
}

static int clamp_q(int v) { return v < -8 ? -8 : (v > 7 ? 7 : v); }

/* std::max(a, b) == (a < b) ? b : a */
static float max_ref(float a, float b) { return (a < b) ? b : a; }

/* Native sidecar packer quantizer: nearbyint under FE_TONEAREST (ties to even).
 * Restates source/q4rdna_sidecar_pack.cpp:126-129. */
int q4o_quantize_value_rne(float value, float scale)
{
    if (scale == 0.0f) return 0;
    return clamp_q(x86_float_to_int(nearbyintf(value / scale)));
}

/* Restates source/q4rdna_sidecar_pack.cpp:131-138 (sequential float sum). */
static float sidecar_scale_error(const float *input, float scale)
{
    float error = 0.0f;
    for (unsigned i = 0; i < Q4O_GROUP; ++i) {
        float delta = scale * (float)q4o_quantize_value_rne(input[i], scale) - input[i];
        error += delta * delta;
    }
    return error;
}

/* Native sidecar packer scale search: starts = {+range, -range} x
 * {1, .9, .8, .7, .6} rounded to fp16, up to 12 least-squares refinements
 * each, first strict minimum wins.  Restates source/q4rdna_sidecar_pack.cpp:140-179
 * (the same algorithm as source/pack_q4rdna_sidecar.py:44-73 with sequential
 * float sums instead of torch reductions). */
uint16_t q4o_select_scale_sidecar(const float *input)
{
    float positive_max = 0.0f, negative_max = 0.0f;
    for (unsigned i = 0; i < Q4O_GROUP; ++i) {
        positive_max = max_ref(positive_max, input[i]);
        negative_max = max_ref(negative_max, -input[i]);
    }
    if (positive_max == 0.0f && negative_max == 0.0f) return 0;
    float a = positive_max / 7.0f, b = negative_max / 8.0f;
    float positive = (a < b) ? b : a;
    float c = positive_max / 8.0f, d = negative_max / 7.0f;
    float negative = -((c < d) ? d : c);
    static const float factors[5] = {1.0f, 0.9f, 0.8f, 0.7f, 0.6f};
    uint16_t best_bits = 0;
    float best_error = INFINITY;
    for (int f = 0; f < 5; ++f) {
        float starts[2] = {positive * factors[f], negative * factors[f]};
        for (int s = 0; s < 2; ++s) {
            uint16_t scale_bits = q4o_f32_to_fp16(starts[s]);
            for (int iteration = 0; iteration < 12; ++iteration) {
                float scale = q4o_fp16_to_f32_ref(scale_bits);
                float error = sidecar_scale_error(input, scale);
                if (error < best_error) { best_error = error; best_bits = scale_bits; }
                float numerator = 0.0f, denominator = 0.0f;
                for (unsigned i = 0; i < Q4O_GROUP; ++i) {
                    int quant = q4o_quantize_value_rne(input[i], scale);
                    numerator += input[i] * (float)quant;
                    denominator += (float)(quant * quant);
                }
                if (denominator == 0.0f) break;
                uint16_t next_bits = q4o_f32_to_fp16(numerator / denominator);
                if (next_bits == scale_bits) break;
                scale_bits = next_bits;
            }
        }
    }
    return best_bits;
}

/* CPU-experiment quantizer: std::round (ties away from zero).
 * Restates source/q4rdna_cpu_experiment.cpp:136-141. */
int q4o_quantize_value_round(float value, float scale)
{
    if (scale == 0.0f) return 0;
    return clamp_q(x86_float_to_int(roundf(value / scale)));
}

/* Squared error of a stored fp16 scale, accumulated in double.
 * Restates source/q4rdna_cpu_experiment.cpp:143-152. */
static double experiment_scale_error(const float *input, uint16_t scale_bits)
{
    float scale = q4o_fp16_to_f32_ref(scale_bits);
    double error = 0.0;
    for (unsigned i = 0; i < Q4O_GROUP; ++i) {
        int quant = q4o_quantize_value_round(input[i], scale);
        double delta = (double)scale * (double)quant - (double)input[i];
        error += delta * delta;
    }
    return error;
}

/* Restates source/q4rdna_cpu_experiment.cpp:154-164. */
static void consider_scale(const float *input, float scale, uint16_t *best_bits, double *best_error)
{
    if (!isfinite(scale)) return;
    uint16_t bits = q4o_f32_to_fp16(scale);
    double error = experiment_scale_error(input, bits);
    if (error < *best_error) { *best_bits = bits; *best_error = error; }
}

/* Least-squares refinement in double plus the two adjacent fp16 magnitudes.
 * Restates source/q4rdna_cpu_experiment.cpp:166-195. */
static void refine_mse_scale(const float *input, float initial_scale, uint16_t *best_bits, double *best_error)
{
    uint16_t scale_bits = q4o_f32_to_fp16(initial_scale);
    for (int iteration = 0; iteration < 12; ++iteration) {
        float scale = q4o_fp16_to_f32_ref(scale_bits);
        consider_scale(input, scale, best_bits, best_error);
        double numerator = 0.0, denominator = 0.0;
        for (unsigned i = 0; i < Q4O_GROUP; ++i) {
            int quant = q4o_quantize_value_round(input[i], scale);
            numerator += (double)input[i] * (double)quant;
            denominator += (double)quant * (double)quant;
        }
        if (denominator == 0.0) break;
        uint16_t next_bits = q4o_f32_to_fp16((float)(numerator / denominator));
        if (next_bits == scale_bits) break;
        scale_bits = next_bits;
    }
    if ((*best_bits & 0x7fffu) != 0 && (*best_bits & 0x7fffu) < 0x7bffu) {
        uint16_t magnitude = *best_bits & 0x7fffu;
        uint16_t sign = *best_bits & 0x8000u;
        consider_scale(input, q4o_fp16_to_f32_ref((uint16_t)(sign | (uint16_t)(magnitude - 1u))), best_bits, best_error);
        consider_scale(input, q4o_fp16_to_f32_ref((uint16_t)(sign | (uint16_t)(magnitude + 1u))), best_bits, best_error);
    }
}

/* Algorithm ids shared with the product library's packer. */
#define Q4O_ALGO_SIDECAR 0
#define Q4O_ALGO_ABSMAX 1
#define Q4O_ALGO_RANGE 2
#define Q4O_ALGO_MSE 3

/* Experiment scale selection: absmax = fp16(max|v|/7); range = better of the
 * two range scales; mse = range plus 12 x 2 refined starts.
 * Restates source/q4rdna_cpu_experiment.cpp:197-237. */
uint16_t q4o_select_scale_experiment(const float *input, int algorithm)
{
    float positive_max = 0.0f, negative_max = 0.0f, max_abs = 0.0f;
    for (unsigned i = 0; i < Q4O_GROUP; ++i) {
        positive_max = max_ref(positive_max, input[i]);
        negative_max = max_ref(negative_max, -input[i]);
        max_abs = max_ref(max_abs, fabsf(input[i]));
    }
    if (max_abs == 0.0f) return 0;
    if (algorithm == Q4O_ALGO_ABSMAX) return q4o_f32_to_fp16(max_abs / 7.0f);
    float a = positive_max / 7.0f, b = negative_max / 8.0f;
    float positive_range_scale = (a < b) ? b : a;
    float c = positive_max / 8.0f, d = negative_max / 7.0f;
    float negative_range_scale = -((c < d) ? d : c);
    uint16_t best_bits = 0;
    double best_error = INFINITY;
    consider_scale(input, positive_range_scale, &best_bits, &best_error);
    consider_scale(input, negative_range_scale, &best_bits, &best_error);
    if (algorithm == Q4O_ALGO_RANGE) return best_bits;
    static const float start_factors[12] = {1.0f, 0.9f, 0.8f, 0.7f, 0.6f, 0.55f,
                                            0.5f, 0.45f, 0.4f, 0.35f, 0.3f, 0.25f};
    for (int f = 0; f < 12; ++f) {
        refine_mse_scale(input, positive_range_scale * start_factors[f], &best_bits, &best_error);
        refine_mse_scale(input, negative_range_scale * start_factors[f], &best_bits, &best_error);
    }
    return best_bits;
}

/* Scale selection by algorithm id. */
uint16_t q4o_select_scale(const float *group, int algorithm)
{
    if (algorithm == Q4O_ALGO_SIDECAR) return q4o_select_scale_sidecar(group);
    return q4o_select_scale_experiment(group, algorithm);
}

/* ------------------------------------------------------------------ */
/* tile layout                                                         */
/* ------------------------------------------------------------------ */

/* Byte offset of the fp16 scale of (row, group) and of the code byte holding
 * k = 64*group + 2*i (low nibble) and 2*i+1 (high nibble).
 * Tile t = (row/32)*G + group, 1088 bytes: 32 fp16 scales then 32x32 code
 * bytes at 64 + 32*i + row%32.  Restates source/q4rdna_sidecar_pack.cpp:268-277
 * (same placement at source/q4rdna_cpu_experiment.cpp:390-399 and the reader
 * at source/q4rdna.cu:346,359,370). */
uint64_t q4o_scale_offset(uint32_t cols, uint32_t row, uint32_t group)
{
    uint64_t groups = cols / Q4O_GROUP;
    uint64_t tile = (uint64_t)(row / Q4O_TILE_ROWS) * groups + group;
    return tile * Q4O_TILE_BYTES + 2u * (row % Q4O_TILE_ROWS);
}

uint64_t q4o_code_offset(uint32_t cols, uint32_t row, uint32_t k)
{
    uint64_t groups = cols / Q4O_GROUP;
    uint32_t group = k / Q4O_GROUP, i = (k % Q4O_GROUP) / 2u;
    uint64_t tile = (uint64_t)(row / Q4O_TILE_ROWS) * groups + group;
    return tile * Q4O_TILE_BYTES + 64u + 32u * i + (row % Q4O_TILE_ROWS);
}

/* Quantize a row-major fp32 matrix [rows][cols] into Q4_RDNA tiles
 * (rows%32 == 0, cols%64 == 0; tiles holds rows*cols*34/64 bytes).
 * The per-group code assignment uses the stored fp16 scale, with the
 * rounding rule of the chosen algorithm family.
 * Restates source/q4rdna_sidecar_pack.cpp:259-279 and
 * source/q4rdna_cpu_experiment.cpp:261-273,387-399. */
int q4o_pack(const float *w, uint32_t rows, uint32_t cols, int algorithm, uint8_t *tiles)
{
    if (rows % Q4O_TILE_ROWS || cols % Q4O_GROUP || algorithm < 0 || algorithm > 3) return -1;
    fesetround(FE_TONEAREST);
    uint32_t groups = cols / Q4O_GROUP;
    for (uint32_t r = 0; r < rows; ++r) {
        for (uint32_t g = 0; g < groups; ++g) {
            const float *values = w + (uint64_t)r * cols + (uint64_t)g * Q4O_GROUP;
            uint16_t scale_bits = q4o_select_scale(values, algorithm);
            float scale = q4o_fp16_to_f32_ref(scale_bits);
            uint64_t so = q4o_scale_offset(cols, r, g);
            tiles[so] = (uint8_t)(scale_bits & 0xffu);
            tiles[so + 1] = (uint8_t)(scale_bits >> 8);
            for (uint32_t i = 0; i < Q4O_GROUP / 2u; ++i) {
                int lo, hi;
                if (algorithm == Q4O_ALGO_SIDECAR) {
                    lo = q4o_quantize_value_rne(values[2 * i], scale);
                    hi = q4o_quantize_value_rne(values[2 * i + 1], scale);
                } else {
                    lo = q4o_quantize_value_round(values[2 * i], scale);
                    hi = q4o_quantize_value_round(values[2 * i + 1], scale);
                }
                tiles[q4o_code_offset(cols, r, g * Q4O_GROUP + 2u * i)] =
                    (uint8_t)((lo & 15) | ((hi & 15) << 4));
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* dequant and GEMV                                                     */
/* ------------------------------------------------------------------ */

/* w = fp32(scale) * float(code), the exact product (signed zero included),
 * as source/q4rdna_cpu_experiment.cpp:264-272 forms it (output[i] =
 * stored_scale * float(low)), over the tile layout above. */
static void dequant_with(const uint8_t *tiles, uint32_t rows, uint32_t cols, float *w,
                         float (*decode)(uint16_t))
{
    for (uint32_t r = 0; r < rows; ++r) {
        for (uint32_t k = 0; k < cols; k += 2) {
            uint64_t so = q4o_scale_offset(cols, r, k / Q4O_GROUP);
            float scale = decode((uint16_t)(tiles[so] | (tiles[so + 1] << 8)));
            uint8_t b = tiles[q4o_code_offset(cols, r, k)];
            w[(uint64_t)r * cols + k] = scale * (float)q4o_nibble_low(b);
            w[(uint64_t)r * cols + k + 1] = scale * (float)q4o_nibble_high(b);
        }
    }
}

/* Runtime semantics: the scale decoded exactly (__half2float). */
void q4o_dequant(const uint8_t *tiles, uint32_t rows, uint32_t cols, float *w)
{
    dequant_with(tiles, rows, cols, w, q4o_fp16_to_f32);
}

/* The CPU experiment's own dequantized values (stored_scale from its fp16
 * decode, which halves subnormal scales): source/q4rdna_cpu_experiment.cpp:264-271. */
void q4o_dequant_ref_cpu(const uint8_t *tiles, uint32_t rows, uint32_t cols, float *w)
{
    dequant_with(tiles, rows, cols, w, q4o_fp16_to_f32_ref);
}

/* Sequential fp32 GEMV: acc = fma(scale*code, x[k], acc) for k = 0..cols-1,
 * per row, acc starting at 0.  Restates source/q4rdna_gemv_bench.hip:189-211
 * for any rows x cols; rows [row_begin, row_end) only.  ref_cpu_decode = 1
 * decodes scales as that file's half_to_float does (:163-187, subnormals
 * halved); 0 decodes them as the GPU kernels do (__half2float). */
void q4o_gemv_seq_f32(const uint8_t *tiles, uint32_t rows, uint32_t cols, const float *x,
                      float *y, uint32_t row_begin, uint32_t row_end, int ref_cpu_decode)
{
    float (*decode)(uint16_t) = ref_cpu_decode ? q4o_fp16_to_f32_ref : q4o_fp16_to_f32;
    uint32_t groups = cols / Q4O_GROUP;
    (void)rows;
    for (uint32_t r = row_begin; r < row_end; ++r) {
        uint32_t rt = r / Q4O_TILE_ROWS, lane = r % Q4O_TILE_ROWS;
        float sum = 0.0f;
        for (uint32_t g = 0; g < groups; ++g) {
            const uint8_t *tile = tiles + ((uint64_t)rt * groups + g) * Q4O_TILE_BYTES;
            float scale = decode((uint16_t)(tile[2 * lane] | (tile[2 * lane + 1] << 8)));
            for (uint32_t i = 0; i < Q4O_GROUP / 2u; ++i) {
                uint8_t packed = tile[64 + i * Q4O_TILE_ROWS + lane];
                sum = fmaf(scale * (float)q4o_nibble_low(packed), x[g * Q4O_GROUP + 2 * i], sum);
                sum = fmaf(scale * (float)q4o_nibble_high(packed), x[g * Q4O_GROUP + 2 * i + 1], sum);
            }
        }
        y[r] = sum;
    }
}

/* The same loop, row tiles spread over OpenMP threads (each row keeps its
 * sequential order, so the result is identical); the CPU baseline's
 * all-cores variant.  Returns the number of threads used. */
int q4o_gemv_seq_f32_mt(const uint8_t *tiles, uint32_t rows, uint32_t cols, const float *x, float *y,
                        int threads)
{
    int used = 1;
    int64_t tiles_n = rows / Q4O_TILE_ROWS;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
    {
#pragma omp single
        used = omp_get_num_threads();
#pragma omp for schedule(static)
        for (int64_t t = 0; t < tiles_n; ++t)
            q4o_gemv_seq_f32(tiles, rows, cols, x, y, (uint32_t)t * Q4O_TILE_ROWS,
                             (uint32_t)(t + 1) * Q4O_TILE_ROWS, 0);
    }
#else
    (void)threads;
    q4o_gemv_seq_f32(tiles, rows, cols, x, y, 0, rows, 0);
#endif
    return used;
}

/* q4o_pack with rows spread over OpenMP threads (every (row, group) is
 * independent, so the bytes are identical to q4o_pack's); the all-cores
 * variant of the packing baseline, as the reference packer parallelises
 * independent groups (source/q4rdna_sidecar_pack.cpp:262).  Returns the
 * number of threads used, or -1 for an unsupported shape or algorithm. */
int q4o_pack_mt(const float *w, uint32_t rows, uint32_t cols, int algorithm, uint8_t *tiles, int threads)
{
    if (rows % Q4O_TILE_ROWS || cols % Q4O_GROUP || algorithm < 0 || algorithm > 3) return -1;
    int used = 1;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
    int64_t blocks = rows / Q4O_TILE_ROWS;
    int bad = 0;
#pragma omp parallel reduction(| : bad)
    {
#pragma omp single
        used = omp_get_num_threads();
#pragma omp for schedule(dynamic, 1)
        for (int64_t b = 0; b < blocks; ++b) {
            /* One row tile at a time through q4o_pack on a view of its rows:
             * a row tile's bytes are one contiguous run of the tensor. */
            uint64_t off = (uint64_t)b * (cols / Q4O_GROUP) * Q4O_TILE_BYTES;
            bad |= q4o_pack(w + (uint64_t)b * Q4O_TILE_ROWS * cols, Q4O_TILE_ROWS, cols, algorithm, tiles + off) != 0;
        }
    }
    if (bad) return -1;
#else
    (void)threads;
    if (q4o_pack(w, rows, cols, algorithm, tiles) != 0) return -1;
#endif
    return used;
}

/* fp64 GEMV over the exactly dequantized weights (products are exact in
 * double), plus the conditioning sum sum_k |w*x| used by the error gate.
 * Rows are spread over OpenMP threads; each row's sums run in k order, so
 * the result does not depend on the thread count. */
void q4o_gemv_f64(const uint8_t *tiles, uint32_t rows, uint32_t cols, const float *x,
                  double *y, double *absdot)
{
    uint32_t groups = cols / Q4O_GROUP;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t rr = 0; rr < (int64_t)rows; ++rr) {
        uint32_t r = (uint32_t)rr;
        uint32_t rt = r / Q4O_TILE_ROWS, lane = r % Q4O_TILE_ROWS;
        double sum = 0.0, asum = 0.0;
        for (uint32_t g = 0; g < groups; ++g) {
            const uint8_t *tile = tiles + ((uint64_t)rt * groups + g) * Q4O_TILE_BYTES;
            double scale = (double)q4o_fp16_to_f32((uint16_t)(tile[2 * lane] | (tile[2 * lane + 1] << 8)));
            for (uint32_t i = 0; i < Q4O_GROUP / 2u; ++i) {
                uint8_t packed = tile[64 + i * Q4O_TILE_ROWS + lane];
                double p0 = scale * q4o_nibble_low(packed) * (double)x[g * Q4O_GROUP + 2 * i];
                double p1 = scale * q4o_nibble_high(packed) * (double)x[g * Q4O_GROUP + 2 * i + 1];
                sum += p0; sum += p1;
                asum += fabs(p0); asum += fabs(p1);
            }
        }
        y[r] = sum;
        if (absdot) absdot[r] = asum;
    }
}

/* SiLU g/(1+exp(-g)) in long double (llama.cpp's ggml_cuda_op_silu_single,
 * applied by source/q4rdna.cu:232,394,470; the llama.cpp source is not part of
 * the reference, so this is the textbook definition). */
double q4o_silu(double g) { return (double)((long double)g / (1.0L + expl(-(long double)g))); }

/* Epilogues of the fused entry points, in fp64 over fp64 GEMV results:
 * add:    y = Wx + add                 (source/q4rdna.cu:231,393,469)
 * swiglu: y = (W_up x) * silu(W_gate x) (source/q4rdna.cu:232,394,470)      */
void q4o_epilogue_add(const double *y, const float *add, uint32_t rows, double *out)
{
    for (uint32_t r = 0; r < rows; ++r) out[r] = y[r] + (double)add[r];
}

void q4o_epilogue_swiglu(const double *up, const double *gate, uint32_t rows, double *out)
{
    for (uint32_t r = 0; r < rows; ++r) out[r] = up[r] * q4o_silu(gate[r]);
}

/* ------------------------------------------------------------------ */
/* sidecar container                                                   */
/* ------------------------------------------------------------------ */

/* 48-byte header "<8sIIIIIIQQ" and 96-byte entries "<64sIIQQQ", little endian.
 * Layout restates source/q4rdna.cu:26-50 / source/q4rdna_sidecar_pack.cpp:23-47
 * / source/pack_q4rdna_sidecar.py:21-23. */
static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
static uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

/* Loader acceptance rules of source/q4rdna.cu:129-155 applied to an in-memory
 * image of `len` bytes.  Returns the entry count (>= 0) when the loader would
 * accept the file, -1 for a bad header, -2 for a truncated index, -3 for an
 * invalid entry, -4 for truncated data (source/q4rdna.cu:163-170 reads
 * data_bytes from data_offset). */
long q4o_validate_sidecar(const uint8_t *image, uint64_t len)
{
    if (len < 48) return -1;
    if (memcmp(image, "Q4RDNA1", 8) != 0) return -1;
    uint32_t version = rd32(image + 8), count = rd32(image + 12), group = rd32(image + 16);
    uint32_t tile_rows = rd32(image + 20), tile_bytes = rd32(image + 24);
    uint64_t data_offset = rd64(image + 32), data_bytes = rd64(image + 40);
    if (version != 1 || group != 64 || tile_rows != 32 || tile_bytes != 1088) return -1;
    if ((uint64_t)count * 96u > len - 48u) return -2;
    for (uint32_t e = 0; e < count; ++e) {
        const uint8_t *p = image + 48 + (uint64_t)e * 96u;
        uint32_t rows = rd32(p + 64), columns = rd32(p + 68);
        uint64_t offset = rd64(p + 72), size = rd64(p + 80);
        if (memchr(p, 0, 64) == NULL || offset < data_offset || offset + size < offset ||
            offset + size > data_offset + data_bytes || rows % 32u != 0 || columns % 64u != 0 ||
            size != (uint64_t)rows * columns * 34u / 64u)
            return -3;
    }
    if (data_offset > len || data_bytes > len - data_offset) return -4;
    return (long)count;
}
