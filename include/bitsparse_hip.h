/*
 * bitsparse_hip.h — C ABI of libbitsparse_hip.so, the MI355X (gfx950) kernels
 * behind the BitSparse activation-compression path.
 *
 * Conventions (all entry points):
 *   - plain C types only: device pointers as void* / typed pointers, sizes as
 *     int64_t, the HIP stream as an opaque void* (hipStream_t; NULL = the
 *     default stream).  No torch or C++ types cross the boundary.
 *   - every call is asynchronous on `stream`, allocates no device memory and
 *     returns an int status: BS_OK, or an error code with a message available
 *     from bs_last_error() (thread local).  Argument checks happen on the
 *     host before anything is enqueued; a failed call enqueues nothing.
 *   - dtype codes are the reference's codec ids (lib_sparse/bitsparse.py:8-18):
 *     0 = bf16, 1 = float8_e4m3fn, 2 = float8_e5m2.
 *   - matrices are dense, row-major, contiguous ([rows, cols], row stride =
 *     cols), as the reference kernels assume (triton_kernels.py:82).
 *   - a matrix handed to the codec, gradient or GEMM entry points holds
 *     fewer than 2^32 elements (M*N, batch_rows*K, K*N), the range of the
 *     uint32 tile prefix; larger shapes return BS_ERR_INVALID.  The
 *     reference's int32 element offsets (triton_kernels.py:80) end its range
 *     at 2^31.
 *
 * Compressed format (reference triton_kernels.py:1-17, bitsparse.py:120-127):
 *   64x64 tiles, T = ceil(M/64)*ceil(N/64), tile t = tm*grid_n + tn;
 *   bitmask  uint8[T*512]: bit (f%8) of byte t*512 + f/8 is [x > 0] for
 *            tile-flat index f = r*64 + c;
 *   prefix   uint32[T+1]: prefix[0] = 0, prefix[t+1] = prefix[t] + nnz(tile t);
 *   vals     element i of tile t sits at vals[*vals_offset + prefix[t] + rank].
 */
#ifndef BITSPARSE_HIP_H
#define BITSPARSE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BS_OK 0
#define BS_ERR_INVALID 1   /* bad argument (shape, dtype, pointer, size) */
#define BS_ERR_HIP 2       /* a HIP runtime call failed                  */

#define BS_DT_BF16 0
#define BS_DT_E4M3FN 1
#define BS_DT_E5M2 2

/* Last error message of the calling thread ("" when none). */
const char* bs_last_error(void);

/* ABI version of this library (bumped when an entry point changes). */
int bs_abi_version(void);

/*
 * Launch timing (no counterpart in the reference: a measurement hook for
 * benchmarks and profilers that need a kernel's own duration on its stream).
 * bs_launch_timing(1) makes every later compress / decompress kernel launch of
 * the calling thread record a pair of library-owned HIP events at the start
 * and end of the kernel itself (hipExtLaunchKernel), so launch gaps between
 * kernels are not counted; bs_launch_timing(0) stops it.  Either call forgets
 * the launches recorded so far.
 * bs_launch_timing_read waits for the recorded launches, writes up to max_n
 * durations (ms) and kinds (0 compress, 1 decompress) in launch order, sets
 * *n_out to the number recorded, and forgets them.  Events are created (not
 * device memory) the first time a pool slot is used and kept by the thread.
 */
int bs_launch_timing(int enable);
int bs_launch_timing_read(float* ms_out, int* kinds_out, int max_n, int* n_out);

/*
 * Streaming-access threshold (no counterpart in the reference: a tuning and
 * test hook).  A kernel whose dense matrix (compress input, decompress
 * output, gradient, amax / quantize input) holds at least this many bytes
 * loads and stores it with the nontemporal hint: nothing of it can stay in
 * the last-level cache for a later kernel, and the hint raises the HBM rate.
 * Smaller matrices keep plain accesses.  Sets the threshold for the process
 * (bytes < 0: the default, 192 MiB, or BITSPARSE_NT_MIN_BYTES from the
 * environment at load time) and returns the previous one.  Results do not
 * depend on it.
 */
int64_t bs_nontemporal_min_bytes(int64_t bytes);

/*
 * Workspace for the single-pass compress (bs_compress) and the fp8 amax
 * (bs_amax): a status word per compress unit plus an amax slot.  It must be
 * zero-filled once before first use; afterwards every call passes an `epoch`
 * that differs from all epochs used with this workspace since it was last
 * zeroed (1, 2, 3, ... up to 2^30-1).  One workspace serves one stream at a
 * time.  Returns the byte size needed for a dense [M, N] input.
 */
int64_t bs_compress_workspace_bytes(int64_t M, int64_t N);
/*
 * Because of the epochs, bs_compress, bs_compress_relu, bs_amax and
 * bs_amax_relu return BS_ERR_INVALID when `stream` is capturing into a HIP
 * graph (a replay would repeat the captured epoch and read the previous
 * replay's status words / amax as current).  Every other entry point can be
 * captured.
 */

/*
 * Single-pass compress of a dense [M, N] activation: bitmask, prefix and
 * the compacted values in one read of `dense` (decoupled look-back across
 * compress units).
 *   in_dtype     dtype of `dense` (0, 1, 2)
 *   quantize     1: `dense` is bf16 and is quantized to e4m3fn on the fly
 *                with scale = max(amax/448, 1e-9), amax taken from the amax
 *                slot that bs_amax wrote with `amax_epoch`; the bitmask and
 *                vals then describe the quantized values; `scale_out` (fp32,
 *                nullable) receives the scale and `dense_q_out` (nullable,
 *                uint8 [M, N]) the quantized dense copy.
 *   vals         value storage (element size 2 for bf16, 1 for fp8/quantize)
 *   vals_capacity elements available in `vals`; elements that would land at
 *                or past it are not written and bit 0 of `*err_flags` is set
 *   vals_offset_in  device int64 (nullable = 0): where this tensor's values
 *                start in `vals` (the TensorBuffer cursor)
 *   align8       1: round the start offset up to a multiple of 8
 *   vals_offset_out device int64 (nullable): receives start + nnz, the next
 *                cursor.  May not alias vals_offset_in.
 *   vals_start_out device int64 (nullable): receives the (aligned) start.
 *   write_vals   0: write only bitmask and prefix (count pass of the
 *                standalone path, values come later from bs_compact_vals)
 *   err_flags    device int32 (nullable), bits OR-ed in on error
 * Replaces lib_sparse/src/functions.py:55-99 (dense_to_tilesparse), which
 * runs triton_kernels.py:67-97 (_tile_pack_kernel), a torch.cumsum
 * (functions.py:38-40) and triton_kernels.py:109-146 (_compact_vals_kernel).
 */
int bs_compress(const void* dense, int in_dtype, int64_t M, int64_t N, int quantize,
                const uint64_t* amax_slot, uint32_t amax_epoch, float* scale_out,
                void* dense_q_out, uint8_t* bitmask, uint32_t* prefix,
                void* vals, int64_t vals_capacity, const int64_t* vals_offset_in,
                int align8, int64_t* vals_offset_out, int64_t* vals_start_out,
                int write_vals, int32_t* err_flags, void* workspace,
                int64_t workspace_bytes, uint32_t epoch, void* stream);

/*
 * bs_compress of relu(preact) with the ReLU fused: `preact` is the
 * pre-activation z (relu(z) > 0 exactly where z > 0, so the bitmask, prefix and
 * values are those of relu(z)); `relu_out` (nullable, may alias `preact` for
 * the reference's in-place z.relu_()) receives relu(z) with the semantics of
 * torch's GPU relu (x <= 0 -> +0, so -0 -> +0; NaN and positives keep their
 * bits).  With quantize, the amax must be
 * that of relu(z) (bs_amax_relu).  Replaces the h = z.relu_() that precedes
 * compress in lib_sparse/layers.py:29,37 and :107,117 (the minimum entry
 * point's "optional fused ReLU").
 */
int bs_compress_relu(const void* preact, int in_dtype, int64_t M, int64_t N, int quantize,
                     const uint64_t* amax_slot, uint32_t amax_epoch, float* scale_out,
                     void* dense_q_out, uint8_t* bitmask, uint32_t* prefix, void* vals,
                     int64_t vals_capacity, const int64_t* vals_offset_in, int align8,
                     int64_t* vals_offset_out, int64_t* vals_start_out, int write_vals,
                     int32_t* err_flags, void* workspace, int64_t workspace_bytes,
                     uint32_t epoch, void* relu_out, void* stream);

/*
 * Up-projection GEMM with the ReLU and the compress fused into its epilogue:
 *     z = bf16(bf16(x @ W^T) + bias),  h = relu(z)   (torch's GPU relu)
 * and h compressed exactly as bs_compress_relu would compress z, in one
 * kernel: h is never read back from HBM.  x: bf16 [M, K] (row stride ldx),
 * W: bf16 [N, K] (row stride ldw), bias: bf16 [N] (nullable: no bias add,
 * one rounding), h_out: bf16 [M, N] (row stride ldh; nullable: h is not
 * written).  Needs M, N > 0, K >= 0, K and N multiples of 8, ldx, ldw, ldh
 * multiples of 8, x, W, h_out and vals 16-byte aligned, and
 * N <= bs_linear_relu_compress_max_n(device).  The values are bf16;
 * vals_capacity, vals_offset_in, align8, vals_offset_out, vals_start_out,
 * err_flags (capacity bits only), workspace (bs_compress_workspace_bytes(M, N))
 * and epoch as for bs_compress (refused while `stream` is capturing).  The
 * fp32 accumulation order is the kernel's own, so z can differ from a
 * library GEMM's in the last bit of some elements; the compressed form is
 * always exactly that of the h it writes.
 *   timeout_flag    nullable int32 the kernel sets to 1 when a look-back wait
 *                   gave up (the compressed form is then wrong and must be
 *                   discarded), with a plain store: device memory, or pinned
 *                   host memory through its device address
 *                   (bs_host_device_pointer), which the host can read once
 *                   the kernel has ended without a copy on the stream.  A
 *                   unit can wait for a workgroup dispatched
 *                   after it in the same 128-row strip, so the strip's
 *                   workgroups must be co-resident: the N bound keeps them to
 *                   half of what the device holds, but other streams' work
 *                   can still crowd them out.
 *   patience_ticks  how long one wait may last, in s_memrealtime ticks
 *                   (100 MHz); < 0: 20 ms; 0: every unit but the first
 *                   gives up without waiting (a test hook: forces the
 *                   time-out path with every wave still ending normally).
 * Replaces z = x @ W1^T; z = z + b1; h = z.relu_(); dense_to_tilesparse(h) in
 * lib_sparse/layers.py:86-89, :29, :37.
 */
int bs_linear_relu_compress(const void* x, int64_t M, int64_t K, int64_t ldx, const void* w, int64_t N,
                            int64_t ldw, const void* bias, void* h_out, int64_t ldh, uint8_t* bitmask,
                            uint32_t* prefix, void* vals, int64_t vals_capacity, const int64_t* vals_offset_in,
                            int align8, int64_t* vals_offset_out, int64_t* vals_start_out, int32_t* err_flags,
                            int32_t* timeout_flag, int64_t patience_ticks, void* workspace,
                            int64_t workspace_bytes, uint32_t epoch, void* stream);
/* Largest N bs_linear_relu_compress accepts on `device` (-1 if the occupancy
 * query fails).  No counterpart in the reference. */
int64_t bs_linear_relu_compress_max_n(int device);
/* Device address of pinned (hipHostMalloc) host memory, for flags a kernel
 * stores into directly (bs_linear_relu_compress's timeout_flag); BS_ERR_HIP if
 * host_ptr is not mapped for the device.  No counterpart in the reference. */
int bs_host_device_pointer(void* host_ptr, void** device_ptr);

/*
 * bs_compress with pack_sbit storage: the values are written straight into
 * the 15/7-bit stream `stream_bytes` (4-byte aligned, stream_nbytes bytes;
 * value i occupies stream bits [i*b, (i+1)*b), LSB first, b = 15 for bf16
 * and 7 for fp8 / quantize) at value index align8(*vals_offset_in), the
 * TensorBuffer cursor rounded up to a multiple of 8 (functions.py:78-81), so
 * no raw staging buffer is written and read back.  Stream bits outside the
 * run keep their values; dwords at or past stream_nbytes/4 are not written
 * and bit 0 of *err_flags is set.  *vals_start_out (nullable) receives the
 * aligned start and *vals_offset_out (nullable) start + nnz.  relu = 1 takes
 * `dense` as the pre-activation, as bs_compress_relu does (relu_out
 * nullable).  M or N = 0 is refused (BS_ERR_INVALID).  Other arguments as
 * for bs_compress.  Replaces lib_sparse/src/functions.py:76-92 with
 * pack_sbit=True, which runs the compaction (triton_kernels.py:109-146) and
 * the bit packer (src/bitpacking.py:58-117) as separate passes.
 */
int bs_compress_packed(const void* dense, int in_dtype, int64_t M, int64_t N, int quantize,
                       const uint64_t* amax_slot, uint32_t amax_epoch, float* scale_out,
                       void* dense_q_out, uint8_t* bitmask, uint32_t* prefix,
                       void* stream_bytes, int64_t stream_nbytes, const int64_t* vals_offset_in,
                       int64_t* vals_offset_out, int64_t* vals_start_out, int32_t* err_flags,
                       void* workspace, int64_t workspace_bytes, uint32_t epoch, int relu,
                       void* relu_out, void* stream);

/*
 * Per-tile bitmask and nonzero counts (int32[T]) of a dense [M, N] input.
 * Replaces lib_sparse/src/triton_operators.py:21-33 (tile_pack) /
 * triton_kernels.py:67-97 (_tile_pack_kernel).
 */
int bs_tile_pack(const void* dense, int in_dtype, int64_t M, int64_t N,
                 int32_t* tile_counts, uint8_t* bitmask, void* stream);

/*
 * prefix[0] = 0, prefix[1..T] = inclusive scan of counts (uint32, wrapping).
 * Replaces lib_sparse/src/functions.py:38-40 (torch.cumsum into prefix).
 */
int bs_prefix_from_counts(const int32_t* tile_counts, int64_t T, uint32_t* prefix,
                          void* stream);

/*
 * Values of tiles [first_tile, first_tile + num_tiles) to
 * vals[*vals_offset + prefix[t] - prefix[first_tile] + rank], using the
 * given bitmask.  Replaces lib_sparse/src/triton_operators.py:108-115
 * (compact_vals, raw mode) / triton_kernels.py:109-146.
 */
int bs_compact_vals(const void* dense, int in_dtype, int64_t M, int64_t N,
                    const uint8_t* bitmask, const uint32_t* prefix, void* vals,
                    int64_t vals_capacity, const int64_t* vals_offset,
                    int64_t first_tile, int64_t num_tiles, int32_t* err_flags,
                    void* stream);

/*
 * Decompress tiles of a row batch into a dense [batch_rows, K] output
 * (row stride K): tile of batch tile-index p is
 * t = (first_m_tile + p / grid_n) * grid_n + p % grid_n.
 *   vals_dtype    stored dtype; vals_numel = elements readable in `vals`
 *   square        0: out has the stored dtype, out = bit ? v : +0
 *                 1: out is bf16, out = k*v*v (bf16 storage: bf16(bf16(k*v)*v);
 *                    fp8 storage: widened to fp32, rounded once)
 *   scale         device fp32 (nullable, only with square): then
 *                 out = bf16(out * bf16(scale*scale)) afterwards
 * Replaces lib_sparse/src/triton_operators.py:118-138 (unpack_batch_) and
 * :141-162 (unpack_relu2_batch_, including its output.mul_(scale**2)) /
 * triton_kernels.py:158-241.
 */
int bs_decompress(const void* vals, int vals_dtype, int64_t vals_numel,
                  const uint8_t* bitmask, const uint32_t* prefix,
                  const int64_t* vals_offset, void* out, int64_t first_m_tile,
                  int64_t grid_n, int64_t K, int64_t batch_rows,
                  int64_t num_tiles_in_batch, int square, float relu2_scale,
                  const float* scale, void* stream);

/*
 * In place on a bf16 [M, N] gradient: grad = bit ? grad : 0.
 * Replaces lib_sparse/src/triton_operators.py:165-175 (mask_with_bitmask_) /
 * triton_kernels.py:251-276.
 */
int bs_relu_grad(void* grad, int64_t M, int64_t N, const uint8_t* bitmask, void* stream);

/*
 * In place on a bf16 [M, N] gradient:
 *   grad = bit ? bf16(grad * (2*k*fp32(r))) : 0, r gathered from vals;
 *   then, when `scale` is given, grad = bf16(grad * bf16(*scale)).
 * Replaces lib_sparse/src/triton_operators.py:178-202 (relu2_grad_sparse_,
 * including its grad.mul_(scale)) / triton_kernels.py:290-330.
 */
int bs_relu2_grad(void* grad, int64_t M, int64_t N, const void* vals, int vals_dtype,
                  int64_t vals_numel, const uint8_t* bitmask, const uint32_t* prefix,
                  const int64_t* vals_offset, float relu2_scale, const float* scale,
                  void* stream);

/*
 * amax(|x|) of a bf16 array into the workspace's amax slot, tagged with
 * `epoch` (NaN propagates).  Replaces the x.abs().max() of
 * lib_sparse/fp8.py:126.
 */
int bs_amax(const void* x, int64_t n, void* workspace, int64_t workspace_bytes,
            uint32_t epoch, void* stream);

/* bs_amax of relu(preact) (bf16), for bs_compress_relu with quantize. */
int bs_amax_relu(const void* preact, int64_t n, void* workspace, int64_t workspace_bytes,
                 uint32_t epoch, void* stream);

/*
 * q = e4m3fn_RNE(fp32(x) / scale), scale = max(amax/448, 1e-9) with amax
 * from the slot bs_amax wrote with `epoch`; scale_out (nullable) gets the
 * scale.  Replaces lib_sparse/fp8.py:123-129 (to_fp8) together with bs_amax.
 */
int bs_quantize_e4m3fn(const void* x, int64_t n, void* q_out, float* scale_out,
                       const void* workspace, int64_t workspace_bytes, uint32_t epoch,
                       void* stream);

/*
 * r <- k * r^2 in place on a bf16 array, rounded as h.square_() then
 * h.mul_(k) round (bf16(bf16(r*r) * k), NaN -> 0x7fc0), and amax|h| into
 * the workspace's amax slot tagged with `epoch` (then bs_quantize_e4m3fn
 * with that epoch gives to_fp8(h)).  Replaces the h.square_(); h.mul_(k)
 * and the amax of to_fp8(h) in the fp8 ReLU^2 forward of
 * lib_sparse/layers.py:103-120 (with fp8.py:123-129).  Refuses graph capture.
 */
int bs_relu2_square_amax(void* r, int64_t n, float k, void* workspace, int64_t workspace_bytes,
                         uint32_t epoch, void* stream);

/*
 * The ReLU^2 layer's compress with its in-place square fused into the ReLU
 * write-back: `preact` (bf16 z) is compressed as bs_compress_relu compresses
 * it (the bitmask, prefix and values of r = relu(z): bf16 values, or e4m3fn
 * codes with quantize = 1 and the amax of r in amax_slot under amax_epoch),
 * and `relu_out` (required, may alias preact) receives bf16(bf16(r*r) * k)
 * (NaN -> 0x7fc0), what h = z.relu_(); h.square_(); h.mul_(k) leaves in z.
 * k must be finite; values go into a buffer (vals, vals_capacity, the
 * cursor as for bs_compress with align8 = 0).  Replaces lib_sparse/
 * layers.py:107-119 (the relu, the compress and the two in-place passes) for
 * raw storage.  Refuses graph capture.
 */
int bs_compress_relu2(const void* preact, int quantize, int64_t M, int64_t N, const uint64_t* amax_slot,
                      uint32_t amax_epoch, float* scale_out, void* dense_q_out, uint8_t* bitmask,
                      uint32_t* prefix, void* vals, int64_t vals_capacity, const int64_t* vals_offset_in,
                      int64_t* vals_offset_out, int32_t* err_flags, void* workspace, int64_t workspace_bytes,
                      uint32_t epoch, void* relu_out, float k, void* stream);

/*
 * amax|bf16(bf16(r*r) * k)| of a tensor r = relu(z) from its amax|r| (the
 * workspace's amax slot under epoch_in, as bs_amax_relu leaves it), written
 * into the slot under epoch_out: for a finite k that map is non-decreasing
 * in r (the square of a bf16 is exact in fp32 and each rounding is
 * monotonic; NaN stays NaN), so the amax of the squared tensor is the image
 * of the amax.  With bs_compress_relu2 it replaces the separate square-and-
 * amax pass (bs_relu2_square_amax) of the fp8 ReLU^2 forward; then
 * bs_quantize_e4m3fn(relu_out, epoch_out) gives to_fp8(h).  One thread,
 * stream-ordered after the compress that reads the slot.  Refuses graph
 * capture.
 */
int bs_amax_relu2_from(void* workspace, int64_t workspace_bytes, uint32_t epoch_in, uint32_t epoch_out,
                       float k, void* stream);

/*
 * out[c * ld_out + r] = in[r * ld_in + c] for an [R, C] byte matrix: the
 * fp8 operand layout change in front of the fp8 GEMM.  Replaces the
 * a.contiguous() / b.T.contiguous().T / a_fp8.T.contiguous() copies of
 * lib_sparse/fp8.py:36-43 and :111 (torch's elementwise float8 copy).
 * Needs C % 16 == 0, R % 4 == 0, ld_in >= C with ld_in % 16 == 0,
 * ld_out >= R with ld_out % 4 == 0, `in` 16-byte and `out` 4-byte aligned;
 * out must not overlap in.
 */
int bs_transpose_u8(const void* in, int64_t R, int64_t C, int64_t ld_in, void* out, int64_t ld_out,
                    void* stream);

/*
 * out[i] = bf16(in[i]) for n e4m3fn codes (exact; NaN codes give 0x7fc0, as
 * torch's float8 -> bfloat16 cast does).  Replaces autograd's cast of the
 * e4m3fn gradients that lib_sparse/fp8.py:105-113 returns for bf16 inputs.
 * in and out 16-byte aligned.
 */
int bs_widen_e4m3fn(const void* in, int64_t n, void* out, void* stream);

/*
 * C[M, N] (bf16, row-major, row stride N) = A @ B, where A is a dense bf16
 * [M, K] matrix and B is a compressed [K, N] activation (vals 16-byte
 * aligned) decoded tile by tile into LDS (never written to HBM dense).
 * A is given in one of two layouts (16-byte aligned, lda % 8 == 0, lda < 2^24):
 *   a_layout = 0: as its transpose At [K, M], m contiguous, row stride
 *                 lda >= M (the MLP backward's A = dY^T, i.e. At = dY); it is
 *                 transposed into the workspace first
 *   a_layout = 1: row-major [M, K], k contiguous, row stride lda >= K,
 *                 K % 8 == 0 (read in place)
 *   square = 0: B = stored bf16 values          (AspB, bf16 storage)
 *   square = 1: B = k*v*v as in bs_decompress   (AspRelu2B), and with
 *               b_scale (fp8 storage) B = bf16(B * bf16(b_scale^2))
 * fp32 MFMA accumulation; small grids split K into fp32 partial sums,
 * reduced in a fixed order.  `workspace` holds the partial sums and the
 * transposed A (bs_gemm_compressed_b_workspace_bytes; 0 = none needed).
 * Replaces lib_sparse/src/sparse_matmul.py:24-28 (AspB) and :109-113
 * (AspRelu2B): unpack to a dense HBM buffer, then torch.matmul.
 */
int64_t bs_gemm_compressed_b_workspace_bytes(int64_t M, int64_t N, int64_t K, int a_layout);
int bs_gemm_compressed_b(const void* A, int64_t M, int64_t K, int64_t lda, int a_layout,
                         const void* vals, int vals_dtype, int64_t vals_numel,
                         const uint8_t* bitmask, const uint32_t* prefix, const int64_t* vals_offset,
                         int64_t N, int square, float relu2_scale, const float* b_scale, void* C,
                         void* workspace, int64_t workspace_bytes, void* stream);

/*
 * fp8 operands: C[M, N] (bf16) = bf16(a_scale * sB * (A @ Bq)), A an e4m3fn
 * [M, K] matrix with device fp32 scale a_scale (to_fp8 output), B a
 * compressed [K, N] activation with fp8 values (vals_dtype 1 or 2, vals
 * 16-byte aligned), decoded tile by tile into LDS:
 *   square = 0: Bq = the stored codes, sB = *b_scale (their scale);
 *   square = 1: Bq, sB = to_fp8(bs_decompress(B, square=1, b_scale)) -- the
 *               bf16 dense k*v*v (times bf16(b_scale^2) when b_scale is not
 *               null), re-quantized with the to_fp8 rule; computed on the
 *               device from the stored codes (no dense operand is formed).
 *               sB is also written to *b_scale_out when not null.
 * A layouts as bs_gemm_compressed_b (a_layout 0: its transpose At [K, M],
 * m contiguous, lda >= M; 1: row-major, lda >= K), any alignment, lda < 2^31.
 * fp32 MFMA accumulation (v_mfma_scale_f32_32x32x64_f8f6f4, unit block
 * scales), scaled once at the end; small grids split K into fp32 partial
 * sums reduced in a fixed order.  `workspace` (256-byte aligned,
 * bs_gemm_compressed_b_fp8_workspace_bytes with the call's `square`) holds
 * the partial sums, A in fragment order, the code table and, for square = 1,
 * the tensor's value run mapped through the code table once (K*N bytes
 * reserved, the run's nnz bytes written), which the GEMM then stages.
 * Replaces, for fp8 storage, lib_sparse/src/sparse_matmul.py:24-28 (AspB)
 * and :109-113 (AspRelu2B): unpack to a dense HBM buffer, re-quantize
 * (fp8.py:123-129) and the scaled fp8 GEMM (fp8.py:25-49).
 */
int64_t bs_gemm_compressed_b_fp8_workspace_bytes(int64_t M, int64_t N, int64_t K, int a_layout, int square);
int bs_gemm_compressed_b_fp8(const void* A, const float* a_scale, int64_t M, int64_t K, int64_t lda,
                             int a_layout, const void* vals, int vals_dtype, int64_t vals_numel,
                             const uint8_t* bitmask, const uint32_t* prefix, const int64_t* vals_offset,
                             int64_t N, int square, float relu2_scale, const float* b_scale, void* C,
                             float* b_scale_out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The two GEMMs above with B's values in a packed stream (pack_sbit storage,
 * the format of bs_pack_bits below) of stream_nbytes bytes, 4-byte aligned;
 * *vals_offset is a value index into the stream.  Everything else as the
 * unpacked entry points.
 *   bs_gemm_compressed_b_packed: bf16 values (vals_dtype 0, 15-bit fields);
 *     a pre-pass unpacks the tensor's run (its nnz values, not a dense B)
 *     to bf16 in the workspace, which the GEMM then stages as stored
 *     values (square = 1 squares them there).  Workspace:
 *     bs_gemm_compressed_b_packed_workspace_bytes (K N bf16 values
 *     reserved for the run).
 *   bs_gemm_compressed_b_fp8_packed: fp8 values (vals_dtype 1 or 2, 7-bit
 *     fields); the pass that maps the codes for square = 1 reads them from
 *     the stream, and for square = 0 the same pass copies them unmapped, into
 *     the workspace run the GEMM stages (the nnz codes, not a dense B).
 *     Workspace: bs_gemm_compressed_b_fp8_workspace_bytes(M, N, K, a_layout,
 *     1) whatever `square`.
 * Replace the pack_sbit branch of the reference's unpack
 * (lib_sparse/src/triton_kernels.py:186-187, load_packed_at_indices of
 * bitpacking.py:37-55) ahead of its GEMM (sparse_matmul.py:24-28, :109-113).
 */
int64_t bs_gemm_compressed_b_packed_workspace_bytes(int64_t M, int64_t N, int64_t K, int a_layout);
int bs_gemm_compressed_b_packed(const void* A, int64_t M, int64_t K, int64_t lda, int a_layout,
                                const void* stream_bytes, int vals_dtype, int64_t stream_nbytes,
                                const uint8_t* bitmask, const uint32_t* prefix, const int64_t* vals_offset,
                                int64_t N, int square, float relu2_scale, const float* b_scale, void* C,
                                void* workspace, int64_t workspace_bytes, void* stream);
int bs_gemm_compressed_b_fp8_packed(const void* A, const float* a_scale, int64_t M, int64_t K, int64_t lda,
                                    int a_layout, const void* stream_bytes, int vals_dtype, int64_t stream_nbytes,
                                    const uint8_t* bitmask, const uint32_t* prefix, const int64_t* vals_offset,
                                    int64_t N, int square, float relu2_scale, const float* b_scale, void* C,
                                    float* b_scale_out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Packed value stream (pack_sbit storage, reference lib_sparse/src/bitpacking.py).
 * Value i of a stream occupies stream bits [i*PB, (i+1)*PB), least significant
 * bit first (byte i*PB/8 holds the low bits); PB = 15 for bf16 and 7 for fp8
 * codes, the low PB bits of the stored value (a ReLU value's sign bit is 0).
 * Storage is a byte array; readers may touch the 4 bytes after the payload
 * (the reference's guard word, bitpacking.py:32-34).
 */

/*
 * Pack raw values raw[0, count) (vals_dtype elements, the compacted output of
 * bs_compress / bs_compact_vals) into stream indices [*start_index,
 * *start_index + count) of `stream_bytes` (4-byte aligned, stream_nbytes
 * bytes).  count = min(*count_ptr, count_max) when count_ptr (device uint32,
 * e.g. prefix + T) is given, else count_max.  Stream bits outside the run
 * keep their values; words past stream_nbytes are not written and bit 0 of
 * *err_flags is set; a negative *start_index sets bit 1.
 * Replaces lib_sparse/src/bitpacking.py:58-117 (_pack_kernel) as launched by
 * triton_operators.py:61-105.
 */
int bs_pack_bits(const void* raw, int vals_dtype, const uint32_t* count_ptr, int64_t count_max,
                 void* stream_bytes, int64_t stream_nbytes, const int64_t* start_index,
                 int32_t* err_flags, void* stream);

/*
 * bs_decompress / bs_relu2_grad reading the values from a packed stream of
 * stream_nbytes bytes; *vals_offset is a value index into the stream.
 * Replace the pack_sbit branches of triton_kernels.py:186-187 and :320-321
 * (load_packed_at_indices, bitpacking.py:37-55).
 */
int bs_decompress_packed(const void* stream_bytes, int vals_dtype, int64_t stream_nbytes,
                         const uint8_t* bitmask, const uint32_t* prefix, const int64_t* vals_offset,
                         void* out, int64_t first_m_tile, int64_t grid_n, int64_t K,
                         int64_t batch_rows, int64_t num_tiles_in_batch, int square,
                         float relu2_scale, const float* scale, void* stream);
int bs_relu2_grad_packed(void* grad, int64_t M, int64_t N, const void* stream_bytes, int vals_dtype,
                         int64_t stream_nbytes, const uint8_t* bitmask, const uint32_t* prefix,
                         const int64_t* vals_offset, float relu2_scale, const float* scale,
                         void* stream);

/*
 * bs_compress_noalloc — no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): bs_compress / bs_compress_relu
 * with the look-back status words and the fp8 amax slot in a library-owned
 * device array (one per GPU, 4 MiB + 6,672 bytes, kept until the process ends)
 * instead of a caller-allocated workspace.  The call allocates nothing.
 *   quantize   1: bf16 input quantized to e4m3fn; the amax pass (of relu(x)
 *              with relu) runs inside the call on the same array
 *   relu       1: `dense` is the pre-activation z, as for bs_compress_relu
 *              (`relu_out` nullable); 0: `relu_out` must be NULL
 * Other arguments as for bs_compress.  Shapes of more than
 * bs_compress_noalloc_max_tiles() = 2^19 tiles are refused (BS_ERR_INVALID).
 * Each call clears the part of the array it uses before its kernels run, so
 * no state carries over and the call can be captured into a HIP graph; but
 * all calls on one GPU share the array, so calls that overlap on one GPU
 * (two streams, two threads) race and must be serialised by the caller.
 */
int bs_compress_noalloc(const void* dense, int in_dtype, int64_t M, int64_t N, int quantize, int relu,
                        float* scale_out, void* dense_q_out, uint8_t* bitmask, uint32_t* prefix,
                        void* vals, int64_t vals_capacity, const int64_t* vals_offset_in, int align8,
                        int64_t* vals_offset_out, int64_t* vals_start_out, int write_vals,
                        int32_t* err_flags, void* relu_out, void* stream);
int64_t bs_compress_noalloc_max_tiles(void);

/*
 * bs_stream_probe — no counterpart in the reference: a measurement kernel, the
 * floor of the codec kernels' HBM access mix.  mode 0 (compress mix): read the
 * [M, N] bf16 matrix `dense` in the compress kernel's load pattern (8 tiles per
 * 512-thread workgroup, nontemporal when `nontemporal`), store one byte per
 * 8-element chunk into `bitmask` (T*512 bytes) and `vals_per_unit` bytes per
 * 8 tiles into `vals` (16-byte stores); mode 1 (decompress mix): read those
 * bitmask and value bytes and write `dense`.  No scan, compaction or gather:
 * the bytes of a compress (decompress) launch with `vals_per_unit` = the
 * mean value bytes of 8 tiles, and nothing else.  M, N multiples of 64, T a
 * multiple of 8, vals_per_unit a multiple of 128 in [0, 65536], `vals_bytes` >=
 * T/8 * vals_per_unit, `bitmask_bytes` >= T*512.
 */
int bs_stream_probe(int mode, void* dense, int64_t M, int64_t N, void* vals, int64_t vals_bytes,
                    int64_t vals_per_unit, uint8_t* bitmask, int64_t bitmask_bytes, int nontemporal,
                    void* stream);

/* Device pointer of the amax slot inside a workspace (for bs_compress). */
const uint64_t* bs_workspace_amax_slot(const void* workspace, int64_t workspace_bytes);

/*
 * Diagnostics counter inside the workspace: number of look-back fallbacks
 * (a unit counted a predecessor itself after waiting for it) since zeroing.
 * Device pointer to a uint32.
 */
const uint32_t* bs_workspace_fallback_counter(const void* workspace, int64_t workspace_bytes);

#ifdef __cplusplus
}
#endif

#endif /* BITSPARSE_HIP_H */
