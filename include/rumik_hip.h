/* rumik_hip.h — C ABI of the MI355X (gfx950) int4 decode hot path.
 *
 * Every entry point takes raw device pointers, sizes, dtype codes and a HIP stream (passed as void*), launches
 * asynchronously on that stream, allocates nothing and never synchronizes, so every call can be captured in a
 * hipGraph. The return value is RK_OK or a negative status (rk_status_string gives the text); invalid arguments
 * are rejected on the host before any launch.
 *
 * Tensor layouts (row-major, contiguous):
 *   int4 weights  q uint8 [N, K/2] (low nibble = even column), scale fp16 [N, K/128], min fp16 [N, K/128];
 *                 w[n,k] = code[n,k] * scale[n,k/128] + min[n,k/128]
 *   int8 weights  q int8 [N, K] (RK_Q_S8) or uint8 = int8 + 128 (RK_Q_U8); one scale per row (fp16 or fp32)
 *   activations   fp16 / bf16 vectors; outputs fp16 / bf16 / fp32
 *
 * bf16 activations into the GEMVs and the prefill product (rk_gemv_int4_g128*, rk_gemv_int8_rows*,
 * rk_mm_int4_g128*) are converted to fp16 for the fp16 dot products / matrix cores. The conversion is exact for
 * magnitudes in fp16's normal range [2^-14, 65504] (bf16's 8-bit significand fits fp16's 11 bits); larger
 * magnitudes become +-inf and smaller ones lose low bits as fp16 subnormals. The activations these kernels take
 * (LayerNorm outputs, SiLU(gate)*up, attention outputs) are far inside that range. The glue kernels keep bf16 values
 * in fp32 (rk_attn_split's scores included), so they have no such limit.
 */
#ifndef RUMIK_HIP_H
#define RUMIK_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden visibility; exactly the functions declared in this header are exported. */
#pragma GCC visibility push(default)

/* dtype codes */
#define RK_F16 0
#define RK_BF16 1
#define RK_F32 2

/* int8 code layouts */
#define RK_Q_S8 0 /* signed int8 codes in [-127, 127] */
#define RK_Q_U8 1 /* uint8 = int8 + 128 (kernels/cuda_gemv.py:234-242 of the reference) */

/* status codes */
#define RK_OK 0
#define RK_ERR_SHAPE (-1)  /* unsupported or inconsistent sizes ("shape") */
#define RK_ERR_BLOCK (-2)  /* unsupported block shape (waves / rows knobs) */
#define RK_ERR_DTYPE (-3)  /* unsupported dtype code */
#define RK_ERR_NULL (-4)   /* a required pointer is NULL */
#define RK_ERR_ALIGN (-5)  /* a pointer is not aligned as the kernel's vector loads need */
#define RK_ERR_LAUNCH (-6) /* the HIP launch itself failed */
#define RK_ERR_SCRATCH (-7) /* the call needs more scratch than the library's fixed array holds */

typedef void* rk_stream_t; /* a hipStream_t; NULL = the default stream */

/* Version of this ABI (bumped when a signature changes). */
int rk_abi_version(void);

/* Text of a status code (static storage). */
const char* rk_status_string(int status);

/* Batch-1 int4 group-128 GEMV: y[n] = sum_k (code[n,k]*scale[n,k/128] + min[n,k/128]) * x[k], fp32 accumulate.
 * Replaces gemv_int4_cuda(x, q, s, m, out, warps, rows) -> gemv_int4 -> launch_int4
 *   (reference kernels/cuda_gemv.py:226-231, :130-136, :117-128) and the Triton fallback gemv_int4
 *   (kernels/int4_gemv.py:84-96).
 * x: [K] fp16/bf16, 16-byte aligned; q: 16-byte aligned; y: [N] of y_dtype.
 * K % 128 == 0 (reference: TORCH_CHECK(... K % GROUP == 0, "shape")) and K <= ~80000 (x is staged in LDS);
 * any N >= 1 (no multiple-of-block rule). The kernel is picked per shape: the matrix-core kernel
 * (rk_gemv_int4_g128_mfma) for N >= 8192 with K <= 4096, the VALU kernel (rk_gemv_int4_g128_valu) otherwise.
 * waves: waves per block (the reference's `warps` knob), in {1,2,4,8,16}; rows: rows per wave (the reference's
 * `rows`), in {1,2,4,8}; 0 = tuned default. Anything else returns RK_ERR_BLOCK ("unsupported block shape"). */
int rk_gemv_int4_g128(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale, const uint16_t* min,
                      void* y, int y_dtype, int N, int K, int waves, int rows, rk_stream_t stream);

/* The matrix-core kernel for any shape: a wave owns a 16-row tile; each v_mfma_f32_16x16x32_f16 takes the
 * exactly dequantized codes as B and x as A. waves above 4 are clamped to 4 per block; rows is validated, unused.
 * Same contract as rk_gemv_int4_g128 (no separate reference counterpart). */
int rk_gemv_int4_g128_mfma(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale,
                           const uint16_t* min, void* y, int y_dtype, int N, int K, int waves, int rows,
                           rk_stream_t stream);

/* The VALU kernel for any shape (v_dot2_f32_f16): `rows` rows per wave, `waves` per block, exactly the
 * reference's (warps, rows) knobs. Same contract as rk_gemv_int4_g128 (no separate reference counterpart). */
int rk_gemv_int4_g128_valu(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale,
                           const uint16_t* min, void* y, int y_dtype, int N, int K, int waves, int rows,
                           rk_stream_t stream);

/* Two independent int4 g128 GEMVs in one launch, y1 = dequant(q1) x1 and y2 = dequant(q2) x2, each with the
 * contract of rk_gemv_int4_g128 (tuned default block shapes): the decode layer's o projection (o = attn @ w_o^T) and
 * down projection (d = act @ w_down^T), which the reference runs as two back-to-back gemv_int4 calls on inputs that
 * are both ready at that point (engine/rumik_fused.py:115-116). One grid: blocks [0, B1) compute y1, the rest y2.
 * Shapes with K1 <= 2048 and 4096 < K2 <= 16384 run as the pair kernel; other shapes as two launches. */
int rk_gemv_int4_g128_pair(const void* x1, int x1_dtype, const uint8_t* q1, const uint16_t* s1, const uint16_t* m1,
                           void* y1, int y1_dtype, int N1, int K1, const void* x2, int x2_dtype, const uint8_t* q2,
                           const uint16_t* s2, const uint16_t* m2, void* y2, int y2_dtype, int N2, int K2,
                           rk_stream_t stream);

/* The engine's input projection with the MLP activation fused (decode glue): q holds n_plain ordinary rows,
 * then `inter` gate rows, then `inter` up rows (the reference's w_in = [q | k | v | gate | up], engine/
 * rumik_int4.py:97), all int4 g128 over one x. Writes y[0 .. n_plain) and act[c] = silu(gate_c) * up_c for
 * c < inter, with gate and up rounded to y_dtype first -- exactly what the GEMV followed by the SiLU·up part of
 * post (reference engine/fused.py:44-84; rk_silu_mul here) produce, in one launch instead of two. Matrix-core
 * kernel; y may be NULL when n_plain == 0. Same x / q / dtype / alignment rules as rk_gemv_int4_g128_mfma. */
int rk_gemv_int4_g128_silu(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale,
                           const uint16_t* min, void* y, void* act, int y_dtype, int n_plain, int inter, int K,
                           int waves, rk_stream_t stream);

/* One decoder layer's four decode projections in ONE launch: y_plain / act exactly as rk_gemv_int4_g128_silu
 * (w_in over x, act = silu(gate) * up with gate and up rounded to y_dtype first), y_o = dequant(w_o) ob and
 * y_down = dequant(w_down) act, where act is the one this launch computes. Replaces the reference's gemv(h, w_in),
 * the MLP part of fused.post, gemv(ob, w_o) and gemv(act, w_down) of one layer (engine/rumik_fused.py:100-101,
 * 115-116) when o's input is already at hand (the benchmark's layer-projection workload). Shapes: w_in
 * [n_plain + 2*inter, H], w_o [H, H], w_down [H, inter], int4 g128 (codes, fp16 scale / min) as rk_gemv_int4_g128;
 * H == 2048; inter a multiple of 128 up to 12288 (at most 48 gate / up pairs per block);
 * n_plain >= 0 with at most 12 rows per block (3072 on 256 CUs); RK_ERR_SHAPE otherwise: then run
 * rk_gemv_int4_g128_silu and rk_gemv_int4_g128_pair. x / ob RK_F16 or RK_BF16 (x_dtype), outputs RK_F16 or RK_BF16
 * (y_dtype); x, ob and the code arrays 16-byte aligned, the scale and min arrays 4-byte aligned (RK_ERR_ALIGN).
 * ws: rk_gemv_int4_g128_layer_ws_bytes(inter) bytes, 4-byte aligned, ZEROED before its first use and then kept
 * for this call alone (its words carry per-block launch counters, so hipGraph replays need no reset; one launch
 * at a time per workspace). One block per CU, all resident at once: the call needs the whole device (256 CUs on
 * MI355X; with fewer CUs, e.g. a partitioned device, every call returns RK_ERR_SHAPE) and no other kernel running
 * on it meanwhile (a block that cannot start leaves the others waiting). The grid meets once (act), every wait
 * bounded: a wait that runs out (200 ms) sets bit 0 of the workspace's first 32-bit word and leaves y_down
 * unwritten; the caller reads that word after the call's stream has finished (LayerProjections.status()) and
 * zeroes it before reusing the workspace. No engine path calls this entry: in the decode step o's input is this
 * layer's attention output, which depends on the q / k / v this launch produces. No separate reference
 * counterpart. */
size_t rk_gemv_int4_g128_layer_ws_bytes(int inter);
int rk_gemv_int4_g128_layer(const void* x, const void* ob, int x_dtype, const uint8_t* q_in, const uint16_t* s_in,
                            const uint16_t* m_in, const uint8_t* q_o, const uint16_t* s_o, const uint16_t* m_o,
                            const uint8_t* q_down, const uint16_t* s_down, const uint16_t* m_down, void* y_plain,
                            void* act, void* y_o, void* y_down, int y_dtype, int n_plain, int inter, int H, void* ws,
                            size_t ws_bytes, rk_stream_t stream);

/* Batch-1 int8 per-row GEMV: y[n] = scale[n] * sum_k code[n,k] * x[k], fp32 accumulate.
 * Replaces gemv_int8_cuda(x, q, s, out) -> gemv_int8 (reference kernels/cuda_gemv.py:245-249, :188-195).
 * q_kind: RK_Q_S8 or RK_Q_U8; scale dtype RK_F16 or RK_F32; y dtype RK_F32 / RK_BF16 / RK_F16.
 * K % 16 == 0, x and q 16-byte aligned; any N >= 1 (the reference needs N % 16 == 0 and K % 512 == 0). */
int rk_gemv_int8_rows(const void* x, int x_dtype, const void* q, int q_kind, const void* scale, int s_dtype,
                      void* y, int y_dtype, int N, int K, rk_stream_t stream);

/* rk_gemv_int8_rows with an explicit block shape: waves per block in {1,2,4,8,16} and rows per wave in
 * {1,2,4,8} (0 = the tuned default; anything else RK_ERR_BLOCK). Same results for every shape; the reference's
 * gemv_int8 has no such knobs (kernels/cuda_gemv.py:188-195), this entry point exists for block-shape sweeps. */
int rk_gemv_int8_rows_ex(const void* x, int x_dtype, const void* q, int q_kind, const void* scale, int s_dtype,
                         void* y, int y_dtype, int N, int K, int waves, int rows, rk_stream_t stream);

/* int4 group-128 matrix product for the prefill: Y[m,n] = sum_k X[m,k] * w[n,k], fp32 accumulate, MFMA.
 * Replaces mm_int4(x, q, s, m) -> _mm_int4 (reference kernels/mm_int4.py:59-73, :24-46).
 * X: [M, K] fp16/bf16 with row stride ldx elements (ldx % 8 == 0, 16-byte aligned rows);
 * Y: [M, N] of y_dtype with row stride ldy. K % 128 == 0; any M >= 1, N >= 1. */
int rk_mm_int4_g128(const void* X, int x_dtype, int ldx, const uint8_t* q, const uint16_t* scale,
                    const uint16_t* min, void* Y, int y_dtype, int ldy, int M, int N, int K, rk_stream_t stream);

/* The kernel plan rk_mm_int4_g128 (use_workspace = 0) or rk_mm_int4_g128_ws (use_workspace = 1) runs for this
 * shape: *kernel = RK_MM_TILE128 (LDS-staged 128 x 128 tiles), RK_MM_TILE64 (LDS-staged 64 x 64 tiles),
 * RK_MM_REGS (register-staged 64 x 64 tiles, for K too long to stage a block's scales in LDS), or, with a
 * workspace only, RK_MM_PREP128 / RK_MM_PREP64 / RK_MM_PREP48 (X prepared once into the workspace in matrix-core
 * fragment order, then blocks of 128 / 64 / 48 rows x 128 columns fed by direct memory-to-LDS copies; chosen when
 * the shape has enough column blocks to fill the chip, K is short enough for a block's scale and min rows to sit
 * in LDS, and N * K / 128 is a multiple of 8; RK_MM_WIDE128 is the same for M > 64 with K / 128 even and >= 4:
 * 128 x 128 blocks of four waves, each owning 64 x 64 of the block, two blocks per CU, split over K (*splits > 1)
 * for M >= 256 with K / 128 > 16 when the tiles are few), or, for
 * M <= 48 and K <= 2048 (with or without a workspace),
 * RK_MM_STREAM (X held in registers as matrix-core fragments for the whole launch while 16-column tiles of codes
 * stream past, one block per CU, no workspace);
 * *splits = the number of K splits (1 = none; > 1 only with a workspace). Host-only query, no GPU needed; RK_ERR_SHAPE for sizes rk_mm_int4_g128 rejects. Part of the
 * mm_int4 drop-in (reference kernels/mm_int4.py:59-73 picks its Triton tile from BM / BN); the reference has no
 * plan query. */
#define RK_MM_REGS 0
#define RK_MM_TILE128 1
#define RK_MM_TILE64 2
#define RK_MM_PREP128 3
#define RK_MM_PREP64 4
#define RK_MM_PREP48 5
#define RK_MM_STREAM 6
#define RK_MM_WIDE128 7
int rk_mm_int4_plan(int M, int N, int K, int use_workspace, int* kernel, int* splits);

/* Bytes of workspace rk_mm_int4_g128_ws uses for this shape (0: it needs none). Shapes whose output tiles alone
 * leave CUs idle (few rows and columns, long K) are split over K into fp32 partial sums that a second kernel adds
 * in a fixed order; shapes on the RK_MM_PREP* kernels hold X prepared in fragment order (ceil(M / 16) * 16 * K
 * fp16) and its per-group row sums (K / 128 * ceil(M / 16) * 16 fp32); so do those on RK_MM_WIDE128, plus
 * splits * M * N fp32 partial sums when split. Part of the same drop-in for mm_int4
 * (reference kernels/mm_int4.py:59-73), which allocates its output per call; the Python wrapper allocates this
 * workspace the same way. */
size_t rk_mm_int4_workspace_bytes(int M, int N, int K);

/* rk_mm_int4_g128 with a caller-provided workspace of at least rk_mm_int4_workspace_bytes(M, N, K) bytes
 * (16-byte aligned; may be NULL when that is 0); RK_ERR_SHAPE if it is smaller. Same results as rk_mm_int4_g128 up
 * to fp32 summation order. Calls that share one workspace must be ordered on one stream. */
int rk_mm_int4_g128_ws(const void* X, int x_dtype, int ldx, const uint8_t* q, const uint16_t* scale,
                       const uint16_t* min, void* Y, int y_dtype, int ldy, int M, int N, int K, void* workspace,
                       size_t workspace_bytes, rk_stream_t stream);

/* rk_mm_int4_g128_ws without a workspace argument and without any allocation: the split-K partial sums go to a
 * fixed array of RK_MM_SCRATCH_BYTES in the library's device memory (one per GPU, held until the process ends,
 * its address looked up once per device on the first call). No counterpart in the reference: it is for callers
 * that cannot allocate (code under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same plan, kernels and results as rk_mm_int4_g128_ws, except that it never takes the RK_MM_PREP* kernels (their
 * prepared X would not fit the array): where rk_mm_int4_g128_ws takes one, this entry runs the tile plan of
 * rk_mm_int4_g128 (results equal up to fp32 summation order). The limit is checked on the plan this entry runs (the
 * tile plan, never a RK_MM_PREP* one): when that plan splits K and its fp32 partial sums (splits * M * N * 4 bytes)
 * exceed RK_MM_SCRATCH_BYTES (no shape with K <= 49152 does), the call returns RK_ERR_SCRATCH before any launch.
 * rk_mm_int4_workspace_bytes may be larger for the same shape (it sizes the prepared-X plan), and such a call still
 * succeeds. Every call on one GPU shares that GPU's array: calls that overlap on one GPU (on different streams
 * without ordering) race and give wrong results; calls ordered on one stream are safe. */
#define RK_MM_SCRATCH_BYTES (8u << 20)
int rk_mm_int4_g128_noalloc(const void* X, int x_dtype, int ldx, const uint8_t* q, const uint16_t* scale,
                            const uint16_t* min, void* Y, int y_dtype, int ldy, int M, int N, int K,
                            rk_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * Decode-step glue (reference engine/fused.py). Activations of one decode step are vectors of `act_dtype`
 * (fp16 or bf16); the KV cache is [NKV, S, HD] per layer in act_dtype; `pos` is an int64 on the device, read by
 * the kernels, so one captured graph serves every sequence length.
 * ------------------------------------------------------------------------------------------------------------ */

/* x = bf16/fp16(emb_q[tok] * emb_s[tok]) (int8 row, fp16 scale); h = LayerNorm(x) * w.
 * Replaces fused.embed_ln (reference engine/fused.py:16-27). tok: int64 on the device. */
int rk_embed_ln(const int64_t* tok, const int8_t* emb_q, const uint16_t* emb_s, const void* ln_w, void* x, void* h,
                int act_dtype, int H, float eps, rk_stream_t stream);

/* x = x + a + b (fp32 sum, one rounding); h = LayerNorm(x) * w (centre, rsqrt(var + eps), no bias).
 * Replaces fused.add_ln (reference engine/fused.py:30-41). b may be NULL (then x = x + a). */
int rk_add_ln(void* x, const void* a, const void* b, const void* ln_w, void* h, int act_dtype, int H, float eps,
              rk_stream_t stream);

/* Everything between the fused projection and attention: interleaved RoPE on the NH query heads (-> q_out) and
 * NKV key heads (-> k cache at slot pos), value heads copied to the v cache, act = silu(gate) * up.
 * y layout [q NH*HD | k NKV*HD | v NKV*HD | gate inter | up inter]; cos/sin tables [S, HD] in act_dtype.
 * rope = 0 skips the rotation (NoPE layers). Replaces fused.post (reference engine/fused.py:44-84). */
int rk_post(const void* y, const int64_t* pos, const void* cos_t, const void* sin_t, void* k_cache, void* v_cache,
            void* q_out, void* act, int act_dtype, int NH, int NKV, int HD, int S, int inter, int rope,
            rk_stream_t stream);

/* Flash-decoding partials over cache slots 0..pos: grid (NKV, nsplit); partial (m, l, acc) per query head and
 * split into pm/pl [NH, nsplit] and po [NH, nsplit, HD] (fp32). Replaces fused.attn_split (engine/fused.py:120-169).
 * HD must be 128. */
int rk_attn_split(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos, float* po, float* pm,
                  float* pl, int act_dtype, int NH, int NKV, int HD, int S, int nsplit, float scale,
                  rk_stream_t stream);

/* Merge the nsplit partials of every head: out = sum_i w_i acc_i / sum_i w_i l_i, w_i = exp(m_i - max m).
 * Replaces fused.attn_combine (reference engine/fused.py:172-187). */
int rk_attn_combine(const float* po, const float* pm, const float* pl, const int64_t* pos, void* out, int act_dtype,
                    int NH, int HD, int nsplit, rk_stream_t stream);

/* act[i] = silu(gate[i]) * up[i] for gate_up = [gate inter | up inter], fp32 math, one rounding: the MLP job of
 * fused.post (reference engine/fused.py:76-84), used between the gate/up and down projections. */
int rk_silu_mul(const void* gate_up, void* act, int act_dtype, int inter, rk_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------
 * The whole decode step in one persistent launch (no reference counterpart as a single kernel: it replaces the
 * ~260 launches of RumikFused._step, engine/rumik_fused.py:97-121, plus the audio head of _logits, :84-89).
 * Hidden size 2048 and head dim 128 are fixed; NH * 128 == 2048; NH / NKV in {1, 2, 4, 8}; inter % 128 == 0 and
 * inter <= 11008; 1 <= n_audio <= 512 * nblocks (RK_ERR_SHAPE otherwise). One block per CU (nblocks = 256 on MI355X, co-residency is checked); block b owns rows
 * [8b, 8b + 8) of the residual stream, the w_in tiles and w_down column slices its `work` row lists, attention
 * split b % nsp of KV head b / nsp (b < NKV * nsp), and the combine of head b / 16 with its w_o slice (rows of
 * group b % 16).
 * Weights are stacked over layers and re-laid out once at load time:
 *   w_in rows are [q | k | v | per 8 MLP channels: 8 gate rows, 8 up rows]; tile T = rows [16T, 16T + 16);
 *   win_t holds, per (layer, tile, 128-column group), the 16 rows x 64 bytes of codes in lane order (lane j + 16s:
 *   row j, bytes [16s, 16s + 16) of the group); win_sm per (layer, tile, wave w = 0..7, row) the two scale |
 *   min << 16 words of wave w's column groups (waves 1..7: 2(w - 1), 2(w - 1) + 1; wave 0: 14, 15);
 *   wd_t holds w_down by 16-column slices: per (layer, slice), 2048 rows x 8 bytes; wd_sm per (layer, group) the
 *   2048 rows' scale | min << 16; wo_q holds w_o per (layer, head h, row group r of 128 rows) as 512 items of 16
 *   bytes (item i: row 128r + i / 4, the codes of columns 128h + 32(i % 4) .. + 32); wo_sm per (layer, row, head)
 *   its scale | min << 16. Block b = (head b / 16, row group b % 16) computes that slice of the o projection.
 * Blocks exchange fp16 values as tagged 32-bit words (value | tag << 16, tag = 1 + (step * 64 + layer) % 65535,
 * step = the block's ctr entry) and poll the words themselves: tx, tq, tkv, top, tdp, tpo (fp16 words) and tml
 * (fp32 m / l | tag << 32). All exchange buffers, ctr and status start at zero; after a nonzero status, re-zero them.
 * status bit 1 = a wait exceeded 200 ms (the step finishes early with garbage); bit 2 = pos outside [0, S)
 * (nothing is computed or written, pos is not advanced); bit 3 = some layer's residual sum x = x + o + down left
 * the fp16 range or was NaN (the step is fp16 end to end, unlike the reference's bf16 engine; the step completes,
 * its outputs are not meaningful). Bit 0 accompanies bit 1.
 * ------------------------------------------------------------------------------------------------------------ */
typedef struct rk_decode_params {
    int L, NH, NKV, inter, S, n_audio, nsp;
    float eps, scale;
    unsigned long long sliding; /* bit l set: RoPE on layer l */
    const int64_t* tok;
    int64_t* pos;
    const int8_t* emb_q;    /* [vocab, 2048] */
    const uint16_t* emb_s;  /* [vocab] fp16 */
    const uint8_t* win_t;   /* [L, n_in/16, 16, 64, 16 B] */
    const uint32_t* win_sm; /* [L, n_in/16, 8 waves, 16 rows, 2] */
    const uint8_t* wo_q;    /* [L, NH, 16, 512, 16 B] */
    const uint32_t* wo_sm;  /* [L, 2048, NH]: scale | min << 16 */
    const uint8_t* wd_t;    /* [L, inter/16, 2048, 8 B] */
    const uint32_t* wd_sm;  /* [L, inter/128, 2048] */
    const uint16_t* ln_w;   /* [L, 2048] fp16 */
    const uint16_t* norm_w; /* [2048] */
    const uint16_t* cos_t;  /* [S, 128] fp16 */
    const uint16_t* sin_t;
    uint16_t* kc;           /* [L, NKV, S, 128] fp16 */
    uint16_t* vc;
    const int8_t* head_q;   /* [n_audio, 2048] */
    const uint16_t* head_s; /* [n_audio] fp16 */
    float* logits;          /* [n_audio] */
    const int16_t* work;    /* [nblocks, 16]: w_in tiles (8, -1 = none), slice begin, slice end, 5 unused */
    uint32_t* tx;           /* [16, 2048]: 16 copies */
    uint32_t* tq;           /* [NH*128] */
    uint32_t* tkv;          /* [2, NKV*128] (k, v of the current layer at pos) */
    uint32_t* top;          /* [nblocks (consumer), NH, 8] o-projection partials */
    uint32_t* tdp;          /* [nblocks (consumer), nblocks (producer), 8] down-projection partials */
    uint32_t* tpo;          /* [NH, nsp, 128] normalized split outputs */
    unsigned long long* tml; /* [NH, nsp, 2] */
    unsigned* ctr;          /* [nblocks] step counters */
    unsigned* status;
    uint16_t* hn;           /* [2048] fp16 final LayerNorm output (the sampler's input), or NULL */
} rk_decode_params;

int rk_decode_step_persistent(const rk_decode_params* params, int nblocks, rk_stream_t stream);

/* sizeof(rk_decode_params) as compiled (for bindings that build the struct by hand) */
int rk_decode_params_size(void);

/* The persistent step's compiled limits, for the host code that builds the work table (no GPU needed).
 *   max_tiles        w_in tiles one block may list (work[b][0 .. max_tiles), -1 = none)
 *   first_pass       the block's first tiles computed and published before its q poll: every q / k / v tile a
 *                    block lists must sit in positions [0, first_pass), else its q poll can wait on a tile that
 *                    is published only after that poll (a circular wait across blocks)
 *   max_slices       w_down 16-column slices per block (work[b][slice_begin_col], work[b][slice_end_col])
 *   work_stride      int16 entries per block row of the work table
 *   slice_begin_col, slice_end_col   the columns of work[b] holding the block's slice range
 *   x_copies         copies of the residual stream in tx
 *   max_splits       attention splits per KV head (nsp)
 *   max_slots_per_split  cached slots one split may cover (S / nsp rounded up must not exceed it)
 * No reference counterpart (the reference's step is separate launches, engine/rumik_fused.py:97-121). */
typedef struct rk_decode_limits {
    int max_tiles, first_pass, max_slices, work_stride, slice_begin_col, slice_end_col, x_copies, max_splits,
        max_slots_per_split;
} rk_decode_limits;

int rk_decode_get_limits(rk_decode_limits* out);

/* ------------------------------------------------------------------------------------------------------------
 * The same decode step as ONE launch with the grid split by role (replaces the same reference code as
 * rk_decode_step_persistent: RumikFused._step, engine/rumik_fused.py:97-121, with _logits :84-89). 256 blocks of
 * 1024 threads (one per CU, co-residency checked). Latency blocks (64, role kind 0, index j): residual rows
 * [32j, 32j + 32), attention split j % (64 / NKV) of KV head g = j / (64 / NKV), the combine of head j / 4 and its
 * o slice for rows [512 (j % 4), + 512). Stream blocks (192, kind 1, index i): MLP slices [sb, se) of 16 channels
 * (their gate / up tiles and w_down columns; a contiguous partition of the inter / 16 slices, at most 4 per block)
 * and int8 head rows i + 192 (w + 16 k). role[b] = {kind, index, sb, se} for block b (sb = se = 0 for latency
 * blocks); every index exactly once. The q/k/v tiles (the first NQT = (NH + 2 NKV) * 8 w_in tiles) are computed
 * where stream_qkv_from says, per step (pos is the same in every block): pos < stream_qkv_from: by the latency
 * blocks, nq = NQT / 64 tiles of latency group g (the blocks of KV head g): entries [nq i, nq i + nq), i = j % (64
 * / NKV), of the group's list [q tiles of heads g REP .. g REP + REP - 1 | k tiles of KV head g | v tiles of KV head
 * g] (REP = NH / NKV, 8 tiles per head), each latency block polling x and running the LayerNorm for them;
 * pos >= stream_qkv_from: by the stream blocks, tiles [i NQT / 192, (i + 1) NQT / 192) after their LayerNorm, the
 * latency blocks then starting each layer at the q poll. Both give bit-identical results (the same tiles and
 * K-split sums); the second is faster at long contexts (RoleDecode switches at pos 384).
 * Shapes: NH * 128 == 2048, NKV 4 or 8, inter a multiple of 128 with at most 4 slices per stream block,
 * 1 <= n_audio <= 192 * 16 * 64; nsp (splits per KV head) <= min(16, 64 / NKV) and S <= nsp * 128; min_chunk (the
 * fewest slots per split) a positive multiple of 8 (RK_ERR_SHAPE / RK_ERR_BLOCK otherwise).
 * Weights as for rk_decode_step_persistent (win_t, wo_q, wd_t, wd_sm, ln_w, norm_w, emb, head unchanged), except
 * win_sm: per (layer, tile, 128-column group, row) the word scale | min << 16, and wo_sm: per (layer, head, row).
 * Exchange buffers have two halves (even / odd layers), all tagged words as for rk_decode_step_persistent:
 *   tx [2][16 copies][2048]; tq [2][NH*128]; tkv [2][2][NKV*128]; tpo [2][NH][nsp][128]; tml [2][NH][nsp][2];
 *   top [2][64 latency blocks][NH][32 rows]; tdp [2][64 latency blocks][192 stream blocks][32 rows].
 * All of them, ctr [256] and status start at zero; after a nonzero status, re-zero them. Status bits as for
 * rk_decode_step_persistent (1 wait timed out, 2 pos outside [0, S), 3 residual beyond the fp16 range).
 * local_xcd = 1: every latency group's blocks share one XCD (the role table gives them equal b % 8, and a launch
 * deals block b to XCD (b + c) % 8, which rk_decode_roles_placement lets the host confirm), so the group's split
 * partials and (latency q/k/v) q / k / v words stay in that XCD's L2 (faster hops); with local_xcd = 0 they are
 * written through to memory like the other exchanges (stream q/k/v words always are). */
typedef struct rk_decode_roles_params {
    int L, NH, NKV, inter, S, n_audio, nsp, min_chunk;
    float eps, scale;
    unsigned long long sliding; /* bit l set: RoPE on layer l */
    const int64_t* tok;
    int64_t* pos;
    const int8_t* emb_q;
    const uint16_t* emb_s;
    const uint8_t* win_t;   /* [L, n_in/16, 16 groups, 64 lanes, 16 B] */
    const uint32_t* win_sm; /* [L, n_in/16, 16 groups, 16 rows] */
    const uint8_t* wo_q;    /* [L, NH, 4 quarters, 2048 items, 16 B] */
    const uint32_t* wo_sm;  /* [L, NH, 2048] */
    const uint8_t* wd_t;    /* [L, inter/16, 2048, 8 B] */
    const uint32_t* wd_sm;  /* [L, inter/128, 2048] */
    const uint16_t* ln_w;   /* [L, 2048] fp16 */
    const uint16_t* norm_w;
    const uint16_t* cos_t;  /* [S, 128] fp16 */
    const uint16_t* sin_t;
    uint16_t* kc;           /* [L, NKV, S, 128] fp16 */
    uint16_t* vc;
    const int8_t* head_q;   /* [n_audio, 2048] */
    const uint16_t* head_s;
    float* logits;
    const int16_t* role;    /* [256, 4] */
    uint32_t* tx;
    uint32_t* tq;
    uint32_t* tkv;
    uint32_t* tpo;
    unsigned long long* tml;
    uint32_t* top;
    uint32_t* tdp;
    unsigned* ctr;
    unsigned* status;
    uint16_t* hn;           /* [2048] fp16 final LayerNorm output, or NULL */
    int local_xcd;          /* 1: latency-group exchanges through the group's XCD L2 (see above) */
    long long stream_qkv_from; /* steps with pos >= this compute q/k/v on the stream blocks, 0: always (see above) */
} rk_decode_roles_params;

int rk_decode_step_roles(const rk_decode_roles_params* params, rk_stream_t stream);

/* xcc[b] = the XCD that block b of a 256-block launch ran on (device int32 [256]; asynchronous on stream). Lets
 * the host confirm the round-robin placement local_xcd relies on (xcc[b] - b constant mod 8). No reference
 * counterpart. */
int rk_decode_roles_placement(int32_t* xcc, rk_stream_t stream);

/* sizeof(rk_decode_roles_params) as compiled */
int rk_decode_roles_params_size(void);

/* the role-split step's compiled limits (host-only query) */
typedef struct rk_decode_roles_limits {
    int blocks, latency_blocks, max_slices, x_copies, max_splits, slots_per_wave, waves;
} rk_decode_roles_limits;

int rk_decode_roles_get_limits(rk_decode_roles_limits* out);

/* pos[0] += 1 on the device (the `self.pos += 1` of the captured step, reference engine/rumik_fused.py:120). */
int rk_pos_advance(int64_t* pos, rk_stream_t stream);

/* ---- prompt prefill (reference RumikFused.prefill, engine/rumik_fused.py:54-78): the glue between its mm_int4
 * products for T rows at once, and the causal attention that replaces its torch fp32 _attend. Activations [T, H]
 * row-major fp16 / bf16 (dt); each stored value is rounded once to dt. */

/* x[t] = dt(emb_q[ids[t]] * emb_s[ids[t]]), h[t] = LayerNorm(x[t]) * ln_w for t < T (the embedding lookup and
 * cohere_ln of rumik_fused.py:58,63, rumik_int4.py:38-43). ids int64 [T] (device); emb int8 [V, H] + fp16 [V]. */
int rk_embed_ln_rows(const int64_t* ids, const int8_t* emb_q, const uint16_t* emb_s, const void* ln_w, void* x,
                     void* h, int dt, int T, int H, float eps, rk_stream_t stream);

/* x[t] = dt(x[t] + a[t] + b[t]), h[t] = LayerNorm(x[t]) * ln_w (rumik_fused.py:74 and the next layer's LN, :63);
 * b may be NULL. */
int rk_add_ln_rows(void* x, const void* a, const void* b, const void* ln_w, void* h, int dt, int T, int H, float eps,
                   rk_stream_t stream);

/* Row t of y [T, ldy] = [q | k | v | gate | up] at position p0 + t: RoPE (interleaved pairs, when rope) on q and k,
 * q -> q_out [T, NH*HD], k / v -> cache slot p0 + t of kc / vc [NKV, S, HD], act [T, inter] = silu(gate) * up
 * (rumik_fused.py:64-71). cos / sin [S, HD] in dt. p0 + T <= S. */
int rk_post_rows(const void* y, int ldy, int p0, const void* cos_t, const void* sin_t, void* kc, void* vc,
                 void* q_out, void* act, int dt, int T, int NH, int NKV, int HD, int S, int inter, int rope,
                 rk_stream_t stream);

/* Causal GQA attention for the prompt on the matrix cores: o[t, h] = softmax(q[t, h] . K[g, 0..p0+t]^T * scale)
 * V[g, 0..p0+t], g = h / (NH / NKV). Replaces _attend (engine/rumik_int4.py:163-171, fp32 scores; here fp32
 * scores and softmax, P in fp16 for the PV product, fp32 accumulation). q, o [T, NH*128] fp16; kc, vc [NKV, S, 128]
 * fp16 (one layer), 16-byte aligned; HD = 128, NH / NKV in {1, 2, 4, 8}, p0 + T <= S. */
int rk_prefill_attn(const void* q, const void* kc, const void* vc, void* o, int dt, int T, int p0, int NH, int NKV,
                    int HD, int S, float scale, rk_stream_t stream);

/* ---- the tail of a decode step: stop predictor + top-k + Gumbel-max sampling + counters
 * (reference engine/sample.py; maths of RumikInt4._logits_and_stop / _pick, engine/rumik_int4.py:174-191).
 * Keys: key = (sortable(bits(logit)) << 32) | index with sortable(b) = b ^ ((b >> 31) & 0x7FFFFFFF), sorted
 * descending (value, then larger index first). Chunks of 512 logits, 32 survivors per chunk, top_k <= 32. */

/* z1[r] = gelu(W1[r] . LayerNorm(h; lnw, lnb, eps) + b1[r]) for r < nz, exact (erf) GELU.
 * Replaces stop_hidden[(nz // 16,)](h, lnw, lnb, w1, b1, z1, eps, H=, ROWS=16) (reference engine/sample.py:34-49).
 * h [H] fp16/bf16/fp32; W1 [nz, H] bf16/fp16 (16-byte aligned) or fp32; lnw, lnb [H], b1 [nz], z1 [nz] fp32. */
int rk_stop_hidden(const void* h, int h_dtype, const float* lnw, const float* lnb, const void* w1, int w1_dtype,
                   const float* b1, float* z1, float eps, int H, int nz, rk_stream_t stream);

/* keys[512c .. 512c + 512) = chunk c's keys sorted descending, c < ceil(nv / 512); logits past nv count as -inf,
 * and index end_idx as -inf while step[0] < min_new.
 * Replaces topk_partial[(nch,)](logits, step, keys, NV, END_IDX, MIN_NEW, CH=512) (reference sample.py:53-61).
 * logits [nv] fp16/bf16/fp32; step int64 [1] (device); keys int64 [ceil(nv / 512) * 512]. */
int rk_topk_partial(const void* logits, int logits_dtype, const int64_t* step, int64_t* keys, int nv, int end_idx,
                    int min_new, rk_stream_t stream);

/* Selects the top 32 of the nch chunks' top-32 lists into scratch[0 .. 32) in descending key order (the rest of
 * scratch is not written; the reference sorts all nc slots, of which its pick and sampler check read the first
 * top_k), samples choice = argmax_{j < topk} (value_j * inv_temp - log(-log(clamp(u_j, 1e-10, 1))))
 * (first maximum), token = ids[index of choice]; token = end_id if (w2 . z1 + b2 > 0 and step >= min_new);
 * out[step] = token, tok[0] = token, step[0] += 1.
 * Replaces pick[(1,)](keys, scratch, u, z1, w2, b2, ids, step, pos, tok, out, inv_temp, END_ID, MIN_NEW, NCH,
 * CH=512, KEEP=32, NC=, TOPK=, NZ=) (reference sample.py:65-93; pos is unused there and not taken here).
 * nc (the reference's candidate-list length): a power of two, nch * 32 <= nc <= 4096 (so nch <= 128);
 * 1 <= topk <= 32; u [>= topk], z1, w2 [nz], b2 [1] fp32;
 * ids, step, tok, out int64 (device). */
int rk_pick(const int64_t* keys, int64_t* scratch, const float* u, const float* z1, const float* w2,
            const float* b2, const int64_t* ids, int64_t* step, int64_t* tok, int64_t* out, float inv_temp,
            int64_t end_id, int min_new, int nch, int nc, int topk, int nz, rk_stream_t stream);

/* rk_stop_hidden + rk_topk_partial + rk_pick in ONE launch (what FusedSampler.__call__ runs, reference
 * engine/sample.py:117-127 launches the three kernels): the last block to finish its stop rows or chunk does the
 * pick. keys / scratch / z1 as above (same contents afterwards); counter: one uint32 of device memory, zero before
 * the first call, left at zero by every call (so a captured graph needs no reset). Calls sharing a counter must not
 * overlap. */
int rk_sample_tail(const void* h, int h_dtype, const float* lnw, const float* lnb, const void* w1, int w1_dtype,
                   const float* b1, const float* w2, const float* b2, float eps, int H, int nz, const void* logits,
                   int logits_dtype, int nv, int end_idx, const float* u, const int64_t* ids, int64_t* step,
                   int64_t* tok, int64_t* out, float inv_temp, int64_t end_id, int min_new, int topk, int64_t* keys,
                   int64_t* scratch, int nc, float* z1, unsigned* counter, rk_stream_t stream);

/* Read-only ceiling (a measurement kernel; replaces the reference's kernels/roofline.py:20-33 `read_only`, which
 * loads an int4 matrix's codes, scales and mins and integer-sums them): reads the three buffers a (na bytes),
 * b (nb), c (nc) as one range of 16-byte items in a single grid-stride pass, with 16-byte nontemporal loads,
 * `unroll` loads in flight per thread (1, 2, 4 or 8), and writes one uint32 per block to sink[blocks]: the wrapping
 * sum of the block's 32-bit words, so the sink's total is the wrapping sum of every word of the three buffers.
 * Sizes must be multiples of 16 and the pointers 16-byte aligned (RK_ERR_SHAPE / RK_ERR_ALIGN);
 * 1 <= blocks <= 65536 (256 threads each). */
int rk_read_only(const void* a, size_t na, const void* b, size_t nb, const void* c, size_t nc, int blocks, int unroll,
                 uint32_t* sink, rk_stream_t stream);

/* rk_read_only with the block size as a knob: threads per block 256, 512 or 1024 (RK_ERR_BLOCK otherwise), for the
 * launch-shape sweep of the ceiling. Same reads and sink as rk_read_only. */
int rk_read_only_ex(const void* a, size_t na, const void* b, size_t nb, const void* c, size_t nc, int threads,
                    int blocks, int unroll, uint32_t* sink, rk_stream_t stream);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* RUMIK_HIP_H */
