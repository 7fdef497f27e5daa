/*
 * CPU restatement of the BitSparse activation-compression path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels in
 * bitsparse_amd/csrc are compared against.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it; the product path never
 * calls it and has no CPU fallback.
 *
 * Plain C99, single-threaded, no dependencies.  Element types are carried as
 * raw bit patterns: bf16 = uint16_t, e4m3fn / e5m2 = uint8_t.
 *
 * Format (reference lib_sparse/src/triton_kernels.py:1-17, bitsparse.py:120-127):
 *   tiles are 64x64, tile id t = tm*grid_n + tn (row-major over the tile grid);
 *   inside a tile the flat index is f = r*64 + c;
 *   bitmask byte t*512 + f/8, bit f%8 (LSB first) is [x > 0];
 *   prefix[0] = 0, prefix[t+1] = prefix[t] + popcount(tile t)   (uint32, wraps);
 *   vals[vals_offset + prefix[t] + rank(t,f)] = x for every set bit, where
 *   rank is the number of set bits before f inside the tile.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

#define OR_TILE 64
#define OR_TILE_NUMEL 4096
#define OR_TILE_BYTES 512

enum { OR_BF16 = 0, OR_E4M3FN = 1, OR_E5M2 = 2 };

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float or_bf16_to_f32(uint16_t b) { return f32_from_bits((uint32_t)b << 16); }

/* fp32 -> bf16, round to nearest even; NaN stays a quiet NaN. */
uint16_t or_f32_to_bf16(float f)
{
    uint32_t u = bits_from_f32(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

/* e4m3fn -> fp32 (exact): bias 7, no infinities, S.1111.111 is NaN. */
float or_e4m3fn_to_f32(uint8_t b)
{
    uint32_t s = (uint32_t)(b >> 7), e = (b >> 3) & 15u, m = b & 7u;
    float v;
    if (e == 15u && m == 7u) return s ? -NAN : NAN;
    if (e == 0u) v = ldexpf((float)m, -9);           /* m * 2^-3 * 2^-6 */
    else v = ldexpf((float)(8u + m), (int)e - 10);   /* 1.m * 2^(e-7)   */
    return s ? -v : v;
}

/* e5m2 -> fp32 (exact): the top byte of an IEEE half. */
float or_e5m2_to_f32(uint8_t b)
{
    uint32_t s = (uint32_t)(b >> 7), e = (b >> 2) & 31u, m = b & 3u;
    float v;
    if (e == 31u) v = m ? NAN : INFINITY;
    else if (e == 0u) v = ldexpf((float)m, -16);
    else v = ldexpf((float)(4u + m), (int)e - 17);
    return s ? -v : v;
}

/*
 * fp32 -> e4m3fn with round-to-nearest-even and no saturation: magnitudes
 * that round above 448 (anything > 464, plus Inf and NaN) become NaN 0x7f.
 * Written from the format definition: the representable grid below 2^-6 is
 * the subnormal spacing 2^-9; above it the spacing is 2^(e-3).
 */
uint8_t or_f32_to_e4m3fn(float f)
{
    uint32_t u = bits_from_f32(f);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint8_t)(sign | 0x7f);       /* NaN */
    float x = f32_from_bits(a);
    if (x > 464.0f) return (uint8_t)(sign | 0x7f);          /* rounds past 448 */
    if (x < 0.015625f) {                                     /* below 2^-6 */
        /* subnormal: q = RNE(x / 2^-9) in [0, 8]; 8 is the smallest normal */
        float t = x * 512.0f;                                /* exact */
        float fl = floorf(t);
        float rem = t - fl;
        uint32_t q = (uint32_t)fl;
        if (rem > 0.5f || (rem == 0.5f && (q & 1u))) q++;
        return (uint8_t)(sign | q);                          /* q==8 -> 0x08 */
    }
    /* normal: exponent e in [1,15], 3 mantissa bits */
    int ex;
    float mant = frexpf(x, &ex);                             /* x = mant*2^ex, mant in [0.5,1) */
    int e = ex - 1 + 7;                                      /* biased exponent */
    float t = ldexpf(mant, 4);                               /* in [8,16): 1.mmm * 8 */
    float fl = floorf(t);
    float rem = t - fl;
    uint32_t q = (uint32_t)fl;                               /* 8..15 */
    if (rem > 0.5f || (rem == 0.5f && (q & 1u))) q++;
    if (q == 16u) { q = 8u; e++; }
    /* e <= 15 guaranteed by x <= 464; e==15,q==15 would be NaN but 464 -> 448 */
    return (uint8_t)(sign | ((uint32_t)e << 3) | (q - 8u));
}

/* ------------------------------------------------------------------------ */
/* element predicates and tile geometry                                      */
/* ------------------------------------------------------------------------ */

/* x > 0 as an IEEE compare: NaN, -0.0 and negatives are false, +denormals true.
 * Reference: triton_kernels.py:86 (tile_flat > 0.0). */
static int is_pos(const void* base, int dtype, int64_t idx)
{
    if (dtype == OR_BF16) return or_bf16_to_f32(((const uint16_t*)base)[idx]) > 0.0f;
    if (dtype == OR_E4M3FN) return or_e4m3fn_to_f32(((const uint8_t*)base)[idx]) > 0.0f;
    return or_e5m2_to_f32(((const uint8_t*)base)[idx]) > 0.0f;
}

static int elem_bytes(int dtype) { return dtype == OR_BF16 ? 2 : 1; }

/* ------------------------------------------------------------------------ */
/* compress                                                                  */
/* ------------------------------------------------------------------------ */

/* Per-tile bitmask and popcount.  Reference: triton_kernels.py:67-97
 * (_tile_pack_kernel); out-of-range elements load as 0 so their bits are 0. */
void or_tile_pack(const void* dense, int dtype, int64_t M, int64_t N,
                  uint8_t* bitmask, int32_t* counts)
{
    int64_t grid_m = (M + 63) / 64, grid_n = (N + 63) / 64;
    for (int64_t tm = 0; tm < grid_m; tm++)
        for (int64_t tn = 0; tn < grid_n; tn++) {
            int64_t t = tm * grid_n + tn;
            uint8_t* bm = bitmask + t * OR_TILE_BYTES;
            int32_t cnt = 0;
            memset(bm, 0, OR_TILE_BYTES);
            for (int r = 0; r < 64; r++) {
                int64_t gr = tm * 64 + r;
                if (gr >= M) break;
                for (int c = 0; c < 64; c++) {
                    int64_t gc = tn * 64 + c;
                    if (gc >= N) break;
                    if (is_pos(dense, dtype, gr * N + gc)) {
                        int f = r * 64 + c;
                        bm[f >> 3] |= (uint8_t)(1u << (f & 7));
                        cnt++;
                    }
                }
            }
            counts[t] = cnt;
        }
}

/* prefix[0] = 0; prefix[1:] = cumsum(counts) in uint32.
 * Reference: functions.py:38-40. */
void or_prefix(const int32_t* counts, int64_t T, uint32_t* prefix)
{
    uint32_t acc = 0;
    prefix[0] = 0;
    for (int64_t t = 0; t < T; t++) { acc += (uint32_t)counts[t]; prefix[t + 1] = acc; }
}

/* Scatter every set-bit element of tiles [first_tile, first_tile+num_tiles)
 * to vals[vals_offset + prefix[t] - prefix[first_tile] + rank].
 * Reference: triton_kernels.py:109-146 (_compact_vals_kernel); the values are
 * copied bit for bit in the input's own dtype. */
void or_compact(const void* dense, int dtype, int64_t M, int64_t N,
                const uint8_t* bitmask, const uint32_t* prefix,
                void* vals, int64_t vals_offset, int64_t first_tile, int64_t num_tiles)
{
    int64_t grid_n = (N + 63) / 64;
    int eb = elem_bytes(dtype);
    for (int64_t k = 0; k < num_tiles; k++) {
        int64_t t = first_tile + k;
        int64_t tm = t / grid_n, tn = t % grid_n;
        int64_t base = (int64_t)prefix[t] - (int64_t)prefix[first_tile] + vals_offset;
        int64_t rank = 0;
        for (int f = 0; f < OR_TILE_NUMEL; f++) {
            if (!((bitmask[t * OR_TILE_BYTES + (f >> 3)] >> (f & 7)) & 1)) continue;
            int64_t gr = tm * 64 + f / 64, gc = tn * 64 + f % 64;
            int64_t dst = base + rank++;
            if (gr < M && gc < N)
                memcpy((char*)vals + dst * eb, (const char*)dense + (gr * N + gc) * eb, eb);
            else
                memset((char*)vals + dst * eb, 0, eb);   /* masked load reads 0 */
        }
    }
}

/* ------------------------------------------------------------------------ */
/* fp8 quantisation (the build's definition of lib_sparse.fp8.to_fp8)        */
/* ------------------------------------------------------------------------ */

/* amax(|x|) over a bf16 array, as fp32 (exact: max of bf16 magnitudes).
 * A NaN anywhere makes the result NaN, as torch's max reduction does.
 * Reference: fp8.py:126 (x.abs().max()). */
float or_amax_bf16(const uint16_t* x, int64_t n)
{
    float m = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float v = fabsf(or_bf16_to_f32(x[i]));
        if (v != v) return NAN;
        if (v > m) m = v;
    }
    return m;
}

/* scale = max(amax / 448, 1e-9) in fp32. Reference: fp8.py:126-127. */
float or_fp8_scale(float amax)
{
    float s = amax / 448.0f;
    return s < 1e-9f ? 1e-9f : s;
}

/* q = e4m3fn_RNE(fp32(x) / scale). Reference: fp8.py:128. */
void or_quantize_bf16_to_e4m3fn(const uint16_t* x, int64_t n, float scale, uint8_t* q)
{
    for (int64_t i = 0; i < n; i++) q[i] = or_f32_to_e4m3fn(or_bf16_to_f32(x[i]) / scale);
}

/* ------------------------------------------------------------------------ */
/* decompress                                                                */
/* ------------------------------------------------------------------------ */

static float load_val_f32(const void* vals, int vdtype, int64_t i)
{
    if (vdtype == OR_BF16) return or_bf16_to_f32(((const uint16_t*)vals)[i]);
    if (vdtype == OR_E4M3FN) return or_e4m3fn_to_f32(((const uint8_t*)vals)[i]);
    return or_e5m2_to_f32(((const uint8_t*)vals)[i]);
}

/*
 * Dense [batch_rows, K] output from tiles of rows [first_m_tile, ...).
 * square == 0: out has the stored dtype and receives the stored bits
 *              (unset bits give +0).           Reference: triton_kernels.py:212-241
 * square == 1: out is bf16 = k*v*v; bf16 storage squares in bf16 ((k*v) then *v,
 *              each rounded to bf16), fp8 storage widens to fp32 first and
 *              rounds once.                    Reference: triton_kernels.py:231-238
 */
void or_unpack(const void* vals, int vdtype, const uint8_t* bitmask, const uint32_t* prefix,
               int64_t vals_offset, void* out, int64_t first_m_tile, int64_t grid_n,
               int64_t K, int64_t batch_rows, int64_t num_tiles, int square, float relu2_scale)
{
    int eb = elem_bytes(vdtype);
    for (int64_t pid = 0; pid < num_tiles; pid++) {
        int64_t row_tile = pid / grid_n, k_tile = pid % grid_n;
        int64_t t = (first_m_tile + row_tile) * grid_n + k_tile;
        int64_t base = (int64_t)prefix[t] + vals_offset;
        int64_t rank = 0;
        for (int f = 0; f < OR_TILE_NUMEL; f++) {
            int bit = (bitmask[t * OR_TILE_BYTES + (f >> 3)] >> (f & 7)) & 1;
            int64_t vi = bit ? base + rank : -1;
            if (bit) rank++;
            int64_t orow = row_tile * 64 + f / 64, ocol = k_tile * 64 + f % 64;
            if (orow >= batch_rows || ocol >= K) continue;
            int64_t o = orow * K + ocol;
            if (!square) {
                if (bit) memcpy((char*)out + o * eb, (const char*)vals + vi * eb, eb);
                else memset((char*)out + o * eb, 0, eb);
            } else {
                uint16_t r = 0;
                if (bit) {
                    if (vdtype == OR_BF16) {
                        float v = load_val_f32(vals, vdtype, vi);
                        float kv = or_bf16_to_f32(or_f32_to_bf16(relu2_scale * v));
                        r = or_f32_to_bf16(kv * v);
                    } else {
                        float v = load_val_f32(vals, vdtype, vi);
                        r = or_f32_to_bf16((relu2_scale * v) * v);
                    }
                }
                ((uint16_t*)out)[o] = r;
            }
        }
    }
}

/*
 * x <- bf16(float(x) * float(bf16(s))) over a bf16 array: PyTorch's in-place
 * multiply of a bf16 CUDA tensor by a 0-dim fp32 CUDA tensor, which loads the
 * scalar through the common (bf16) dtype.  Used for output.mul_(scale**2)
 * (triton_operators.py:160-161) and grad.mul_(scale) (:200-201).
 */
void or_bf16_mul_scalar_tensor(uint16_t* x, int64_t n, float s)
{
    float sb = or_bf16_to_f32(or_f32_to_bf16(s));
    for (int64_t i = 0; i < n; i++) x[i] = or_f32_to_bf16(or_bf16_to_f32(x[i]) * sb);
}

/* ------------------------------------------------------------------------ */
/* gradients                                                                 */
/* ------------------------------------------------------------------------ */

/* grad <- bit ? grad : 0 in place over the bf16 [M, N] gradient.
 * Reference: triton_kernels.py:251-276. */
void or_relu_grad(uint16_t* grad, int64_t M, int64_t N, const uint8_t* bitmask)
{
    int64_t grid_n = (N + 63) / 64;
    for (int64_t i = 0; i < M; i++)
        for (int64_t j = 0; j < N; j++) {
            int64_t t = (i / 64) * grid_n + j / 64;
            int f = (int)((i % 64) * 64 + j % 64);
            if (!((bitmask[t * OR_TILE_BYTES + (f >> 3)] >> (f & 7)) & 1)) grad[i * N + j] = 0;
        }
}

/*
 * grad <- bit ? bf16(fp32(grad) * (2*k*fp32(r))) : 0 in place, r gathered from
 * vals; afterwards, when `scale` is given (fp8 storage), grad <- grad * scale
 * with the 0-dim-tensor semantics above.
 * Reference: triton_kernels.py:290-330, triton_operators.py:200-201.
 */
void or_relu2_grad(uint16_t* grad, int64_t M, int64_t N, const void* vals, int vdtype,
                   const uint8_t* bitmask, const uint32_t* prefix, int64_t vals_offset,
                   float relu2_scale, const float* scale)
{
    int64_t grid_m = (M + 63) / 64, grid_n = (N + 63) / 64;
    for (int64_t tm = 0; tm < grid_m; tm++)
        for (int64_t tn = 0; tn < grid_n; tn++) {
            int64_t t = tm * grid_n + tn;
            int64_t base = (int64_t)prefix[t] + vals_offset, rank = 0;
            for (int f = 0; f < OR_TILE_NUMEL; f++) {
                int bit = (bitmask[t * OR_TILE_BYTES + (f >> 3)] >> (f & 7)) & 1;
                float r = 0.0f;
                if (bit) r = load_val_f32(vals, vdtype, base + rank++);
                int64_t gr = tm * 64 + f / 64, gc = tn * 64 + f % 64;
                if (gr >= M || gc >= N) continue;
                uint16_t* g = grad + gr * N + gc;
                if (!bit) { *g = 0; continue; }
                float d = (2.0f * relu2_scale) * r;
                *g = or_f32_to_bf16(or_bf16_to_f32(*g) * d);
            }
        }
    if (scale) or_bf16_mul_scalar_tensor(grad, M * N, *scale);
}

/* ------------------------------------------------------------------------ */
/* one-call compress used as the CPU baseline (same work as the GPU kernel)  */
/* ------------------------------------------------------------------------ */

/* Full compress: bitmask + prefix + vals (vals sized >= nnz). Returns nnz. */
int64_t or_compress(const void* dense, int dtype, int64_t M, int64_t N,
                    uint8_t* bitmask, uint32_t* prefix, int32_t* counts_scratch,
                    void* vals, int64_t vals_offset)
{
    int64_t T = ((M + 63) / 64) * ((N + 63) / 64);
    or_tile_pack(dense, dtype, M, N, bitmask, counts_scratch);
    or_prefix(counts_scratch, T, prefix);
    or_compact(dense, dtype, M, N, bitmask, prefix, vals, vals_offset, 0, T);
    return (int64_t)prefix[T];
}

/* ------------------------------------------------------------------------ */
/* packed value stream (pack_sbit)                                          */
/* ------------------------------------------------------------------------ */

/*
 * Pack raw[0, n) (bf16 uint16 or fp8 uint8 bit patterns, low `bits` bits
 * each) into the byte stream at value index `start`: one output byte at a
 * time, its bits gathered from the (at most two) values overlapping it, bytes
 * shared with bits outside the run merged with their old content.  Follows
 * reference lib_sparse/src/bitpacking.py:58-117 (_pack_kernel: relative_bit,
 * value0 >> bit_offsets | value1 << (bits - bit_offsets), valid_lo/valid_hi
 * merge).
 */
void or_pack_bits(const void* raw, int vdtype, int64_t n, int bits, uint8_t* stream, int64_t start)
{
    if (n <= 0) return;
    int64_t start_bit = start * bits, end_bit = start_bit + n * bits;
    int64_t first_byte = start_bit / 8, end_byte = (end_bit + 7) / 8;
    for (int64_t ob = first_byte; ob < end_byte; ob++) {
        int64_t relative_bit = ob * 8 - start_bit;
        int64_t source_bit = relative_bit > 0 ? relative_bit : 0;
        int64_t idx = source_bit / bits, off = source_bit % bits;
        uint32_t v0 = 0, v1 = 0;
        if (idx < n) v0 = vdtype == OR_BF16 ? ((const uint16_t*)raw)[idx] : ((const uint8_t*)raw)[idx];
        if (idx + 1 < n) v1 = vdtype == OR_BF16 ? ((const uint16_t*)raw)[idx + 1] : ((const uint8_t*)raw)[idx + 1];
        uint32_t mask = (1u << bits) - 1u;
        v0 &= mask;
        v1 &= mask;
        uint32_t packed = (v0 >> off) | (v1 << (bits - off));
        packed = (packed << (relative_bit < 0 ? -relative_bit : 0)) & 0xffu;
        int64_t lo = start_bit - ob * 8, hi = end_bit - ob * 8;
        lo = lo < 0 ? 0 : (lo > 8 ? 8 : lo);
        hi = hi < 0 ? 0 : (hi > 8 ? 8 : hi);
        uint32_t valid = ((1u << hi) - 1u) & ~((1u << lo) - 1u);
        stream[ob] = (uint8_t)((stream[ob] & ~valid) | (packed & valid));
    }
}

/* Value `idx` of a packed stream: two little-endian uint16 words, shifted
 * and masked (reference bitpacking.py:37-55, load_packed_at_indices). */
uint32_t or_unpack_bits_at(const uint8_t* stream, int bits, int64_t idx)
{
    int64_t word = (idx * bits) / 16, shift = (idx * bits) % 16;
    uint32_t w0 = (uint32_t)stream[2 * word] | ((uint32_t)stream[2 * word + 1] << 8);
    uint32_t w1 = (uint32_t)stream[2 * word + 2] | ((uint32_t)stream[2 * word + 3] << 8);
    return ((w0 | (w1 << 16)) >> shift) & ((1u << bits) - 1u);
}
