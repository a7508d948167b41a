/*
 * mxdecode - MI355X (gfx950) decode-step hot path: weight-only int8 linear
 * layers, paged-attention decode and the per-layer glue around them (KV append,
 * rotary embedding, residual + RMSNorm, SwiGLU). C ABI of libmxdecode.so.
 *
 * Conventions
 *   - fp16 tensors are passed as `uint16_t*` (IEEE binary16 bit patterns).
 *   - Every buffer is caller-owned device memory. No call allocates, frees or
 *     synchronises. Work is enqueued on `stream` (a hipStream_t passed as
 *     `void*`; NULL means the legacy default stream).
 *   - Return value: MX_OK (0) or a negative mx_status. The message of the
 *     last failure on the calling thread is returned by mx_last_error().
 *     Nothing throws or aborts across this boundary.
 *   - Strides are in elements.
 */
#ifndef MXDECODE_H
#define MXDECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MX_ABI_VERSION 18

typedef enum mx_status {
    MX_OK = 0,
    MX_ERR_INVALID = -1,     /* bad shape, stride or argument value */
    MX_ERR_UNSUPPORTED = -2, /* valid but outside the supported envelope */
    MX_ERR_ALIGNMENT = -3,   /* pointer or stride not suitably aligned */
    MX_ERR_NULL = -4,        /* required pointer is NULL */
    MX_ERR_LAUNCH = -5,      /* HIP launch error */
    MX_ERR_WORKSPACE = -6    /* workspace missing or too small */
} mx_status;

/* ABI version of the loaded library (MX_ABI_VERSION at build time). */
int mx_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* mx_last_error(void);

/* ----------------------------------------------------------------------------
 * Weight-only int8 linear (W8A16).
 *
 * Replaces the reference's quantized-linear slot: the autoawq WQLinear module
 * that runtime/phase2/worker_server.py:194-205 loads for PHASE2_QUANT=int4, i.e.
 * the nn.Linear contract y[..., N] = x[..., K] W^T (+ b) of every decoder-layer
 * projection (worker_server.py:199-203: the HF decoder layer calls
 * q/k/v/o/gate/up/down_proj). The int8 format itself is defined by this
 * build (per-output-channel symmetric absmax, fp16 scales); see
 * oracle/int8_quant.py for the exact formula and the packed tile layout.
 * ------------------------------------------------------------------------- */

/* Quantize fp32 weights w[N, K] (row stride K) to int8 q[N, K] and fp16
 * scales s[N]. Bit-exact with the CPU restatement. Reference: the slot's
 * model-load step, runtime/phase2/worker_server.py:194-205. */
int mx_w8a16_quantize(const float* w, int64_t N, int64_t K, int8_t* q, uint16_t* scale, void* stream);

/* Pack q[N, K] (int8, row stride K) into the 1 KiB tile layout read by
 * mx_w8a16_linear (N % 16 == 0, K % 64 == 0; N*K bytes): 16 x 64 tiles,
 * k-major (tile (nt, kt) at byte (kt*N/16 + nt)*1024). Bit-exact.
 * Reference: same load step, worker_server.py:194-205. */
int mx_w8a16_pack(const int8_t* q, int64_t N, int64_t K, uint8_t* packed, void* stream);

/* Workspace bytes mx_w8a16_linear needs for this shape (0: none). */
size_t mx_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* y[m, n] = fp16( scale[n] * sum_k x[m, k] * q[n, k] + bias[n] ), fp32
 * accumulation. x: fp16 [M, K] with row stride x_stride (16-byte aligned rows);
 * packed: from mx_w8a16_pack; scale: fp16 [N]; bias: fp16 [N] or NULL;
 * y: fp16 [M, N] with row stride y_stride. Replaces the forward of the
 * reference's quantized linear (autoawq WQLinear.forward, reached from the HF
 * decoder layer; worker_server.py:194-205) and of nn.Linear on the decode path
 * (worker_server.py:773). */
int mx_w8a16_linear(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride, const uint8_t* packed,
                    const uint16_t* scale, const uint16_t* bias, uint16_t* y, int64_t N, int64_t y_stride,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Number of K splits the MFMA path uses for this shape (1 <= M <= 128): 1 means
 * mx_w8a16_linear writes y directly; above 1, mx_w8a16_linear_partials can
 * hand the split partials to a consumer that sums them itself (the decode
 * glue kernels below), saving mx_w8a16_linear's separate reduce launch.
 * Returns 1 for M > 128, where no partials entry exists (mx_w8a16_linear runs
 * 128-row chunks, each planned as M = 128). */
int mx_w8a16_splits(int64_t M, int64_t N, int64_t K);

/* The split-K part of mx_w8a16_linear without the reduction:
 * partials[s][m][n] = scale[n] * sum over the k of split s of x[m, k] q[n, k]
 * (fp32, no bias), for s < mx_w8a16_splits(M, N, K) > 1; partials is fp32
 * [splits][M][N], contiguous. Summing the splits, adding the bias and rounding
 * to fp16 gives mx_w8a16_linear's y. Shapes with one split are rejected
 * (MX_ERR_UNSUPPORTED). No reference counterpart: the reference runs its
 * linear as one HF module call (worker_server.py:194-205). */
int mx_w8a16_linear_partials(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride, const uint8_t* packed,
                             const uint16_t* scale, int64_t N, float* partials, size_t partials_bytes, void* stream);

/* mx_w8a16_linear / mx_w8a16_linear_partials with the SwiGLU product as x:
 * x[m, k] = fp16(fp16(silu(gate_up[m, k])) * gate_up[m, K + k]) for k < K,
 * formed while the kernel stages x (gate_up: fp16 [M, 2K], row stride
 * gu_stride >= 2K). The MLP's down projection of a gate||up projection
 * (transformers' down_proj(act_fn(gate_proj(x)) * up_proj(x)), reached from
 * worker_server.py:771-775) without materialising the product. Requires
 * 4 < M <= 128 (the MFMA path); smaller batches use mx_silu_mul and
 * mx_w8a16_linear. */
int mx_w8a16_linear_swiglu(const uint16_t* gate_up, int64_t M, int64_t K, int64_t gu_stride, const uint8_t* packed,
                           const uint16_t* scale, const uint16_t* bias, uint16_t* y, int64_t N, int64_t y_stride,
                           void* workspace, size_t workspace_bytes, void* stream);
int mx_w8a16_linear_partials_swiglu(const uint16_t* gate_up, int64_t M, int64_t K, int64_t gu_stride,
                                    const uint8_t* packed, const uint16_t* scale, int64_t N, float* partials,
                                    size_t partials_bytes, void* stream);

/* gate||up projection with the SwiGLU product in its epilogue:
 * y[m, c] = fp16(fp16(silu(g)) * u), g = fp16(x W_gate[c]^T (+ b)), u likewise
 * with W_up[c], for c < I; y is fp16 [M, I] (row stride y_stride). The packed
 * weight is the [2I, K] matrix whose rows alternate in groups of 8: rows
 * 16t + [0, 8) = gate rows 8t + [0, 8), rows 16t + [8, 16) = up rows
 * 8t + [0, 8) (scale and bias reordered the same way), quantized and packed
 * as usual. Replaces transformers' act_fn(gate_proj(x)) * up_proj(x) (reached
 * from worker_server.py:771-775) with one launch and half the output bytes.
 * Rows are processed 128 at a time: the VALU GEMV where mx_w8a16_linear would
 * take it (M <= 4 on shapes that split), else one MFMA launch that never splits
 * K, whatever mx_w8a16_splits reports for the plain projection. */
int mx_w8a16_gateup_swiglu(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride, const uint8_t* packed,
                           const uint16_t* scale, const uint16_t* bias, uint16_t* y, int64_t I, int64_t y_stride,
                           void* stream);

/* The whole int8 MLP in one launch: act = mx_w8a16_gateup_swiglu(x) (fp16
 * [M, I], row stride act_stride) and partials = the split-K partials of
 * act Wd^T exactly as mx_w8a16_linear_partials(act, ..., N) writes them
 * (mx_w8a16_splits(M, N, I) slices of [M, N]), both bit-identical to those two
 * calls. Replaces transformers' down_proj(act_fn(gate_proj(x)) * up_proj(x))
 * (reached from worker_server.py:771-775, its linears in the quantized slots
 * of worker_server.py:194-205), which launches each projection in turn; here
 * down's first weight loads overlap the end of gate||up. Takes 4 < M <= 32
 * where gate||up runs unsplit and down splits K in k parts
 * (mx_w8a16_mlp_fused_supported: the Llama-3-8B MLP at batch 32), with act
 * 128-byte aligned and act_stride a multiple of 64; MX_ERR_UNSUPPORTED
 * otherwise, or where the device cannot hold every workgroup of the launch at
 * once. sync: 64 int32 words of device memory, zero before the first call;
 * every call leaves words 0-32 zero again and ORs error bits into word 33
 * (1: a wait for the activations gave up after tens of milliseconds, the
 * outputs then undefined). One call at a time per sync buffer. Measured on
 * MI355X at the Llama-3-8B MLP's 32 rows it is slower than the two calls
 * (48-50 against 39.6-41.3 us): down waits for gate||up's slowest workgroups. */
int mx_w8a16_mlp_fused_supported(int64_t M, int64_t K, int64_t I, int64_t N);
int mx_w8a16_mlp_fused_partials(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride,
                                const uint8_t* gu_packed, const uint16_t* gu_scale, const uint16_t* gu_bias,
                                int64_t I, uint16_t* act, int64_t act_stride, const uint8_t* down_packed,
                                const uint16_t* down_scale, int64_t N, float* partials, size_t partials_bytes,
                                int32_t* sync, void* stream);

/* ----------------------------------------------------------------------------
 * Paged-attention decode.
 *
 * Replaces paged_attention_decode_batched
 * (runtime/phase2/paged_attention_triton.py:745-775) and the Triton kernels it
 * dispatches to: _paged_attn_decode_direct_batched_kernel (:148-243),
 * _paged_attn_decode_split_kernel (:245-336), _paged_attn_decode_direct_kernel
 * (:338-412) and _paged_attn_combine_kernel (:414-457).
 *
 * q:   fp16 (or bf16, MX_PA_BF16) [B, Hq, D] with strides (q_sb, q_sh, 1) (the [B,Hq,1,D] query)
 * k,v: fp16 (bf16) per-layer pool views [num_blocks, Hkv, block_size, D] with strides
 *      (kv_sblk, kv_shead, D, 1) (GpuKVBlockPool.k_layer_view,
 *      runtime/phase2/paged_kv_kernel.py:124-134)
 * block_tables: int32 [B, max_blocks] with row stride bt_sb; entries past a
 *      row's ceil(seq_len / block_size) blocks are never read
 * seq_lens: int32 [B], KV length including the current token
 *      (paged_attention_triton.py:43-50); the kernel reads
 *      min(ceil(seq_len / block_size), max_blocks) blocks; seq_len <= 0 gives
 *      a zero output row
 * out: fp16 (bf16) [B, Hq, D] with strides (o_sb, o_sh, 1)
 * num_pool_blocks: block ids outside [0, num_pool_blocks) are skipped and
 *      recorded in the workspace error word (see mx_paged_attn_error_offset)
 * chunk_tokens: split granularity. All (sequence, kv-head) tiles of 16 tokens
 *      form one sequence that is cut into W equal ranges, one per wave, so
 *      every wave streams the same K/V bytes whatever the mix of lengths.
 *      chunk_tokens > 0 (a multiple of 16, at most 1024) sets ranges of about
 *      that many tokens when every row is at the table width
 *      (max_blocks * block_size); 0 picks 2048 waves (one round of resident
 *      waves on MI355X), fewer when ranges would be shorter than 4 tiles. A
 *      range never exceeds 64 tiles (more waves are used instead). Must be
 *      the value the workspace was sized for. A
 *      second, small kernel on the same stream merges the ranges of a
 *      sequence that more than one wave touched.
 * flags: an OR of MX_PA_SHARED_BLOCKS, MX_PA_BF16 and one of MX_PA_PLAN_WRITE /
 *      MX_PA_PLAN_READ (or 0).
 *      MX_PA_BF16: q, K, V and out hold bf16 instead of fp16 (the same layouts;
 *      scores, softmax and accumulation stay fp32, probabilities enter P.V in
 *      bf16). The reference kernel takes the pool's dtype
 *      (paged_attention_triton.py:500,533-535).
 *      MX_PA_SHARED_BLOCKS: without it K and V are read with the
 *      streaming (non-temporal) cache policy, right when each block id occurs
 *      in one row of block_tables. Set it when rows alias blocks (a shared
 *      prefix): the default policy then keeps a group's repeated reads of the
 *      same blocks in L2 / MALL. Results are the same either way. No reference
 *      counterpart: the reference copies prefix blocks per request
 *      (runtime/phase2/worker_server.py:1442-1449), so its rows never alias.
 *      MX_PA_PLAN_WRITE / MX_PA_PLAN_READ (block_size >= 16, without
 *      MX_PA_SHARED_BLOCKS): a decode step calls attention once per layer with
 *      the same seq_lens, block_tables and shape. A PLAN_WRITE call also records
 *      each wave's tiles (block id, sequence, kv-head, tile) in the workspace; a
 *      later PLAN_READ call with the same workspace starts from that record
 *      instead of locating its range from seq_lens and reading block_tables,
 *      one dependent memory round trip less. Results are identical to a call
 *      without the flags when seq_lens and block_tables are unchanged since
 *      the PLAN_WRITE call (other inputs, such as q and the layer's K/V views,
 *      may differ). Otherwise the output is undefined, no access leaves the
 *      pool, q, out or the workspace, and mismatching pieces set bit 3 (value
 *      8) of the error word. No reference counterpart: the reference re-derives
 *      its grid per layer (paged_attention_triton.py:460-552).
 * Supported: D in {64, 128}; block_size in {4, 8, 16, 32}; Hq = G * Hkv, any G >= 1
 * (G > 8 runs as vg virtual kv-heads of G / vg <= 8 query heads each, vg the smallest
 * such divisor of G; each reads its pool head's K/V, so K/V bytes are read vg times).
 * The workspace holds the split partials (per piece: fp32 m and l, and its
 * output normalised by l in the element type), the tile plan (16 bytes per tile
 * slot, 64 slots and a header per wave, block_size >= 16) and the error word; zero it once at
 * allocation so the error word starts clear. Concurrent calls must not share
 * a workspace. out rows must be 16-byte aligned (o_sb, o_sh multiples of 8).
 * ------------------------------------------------------------------------- */
#define MX_PA_SHARED_BLOCKS 1u
#define MX_PA_BF16 2u
#define MX_PA_PLAN_WRITE 4u
#define MX_PA_PLAN_READ 8u

size_t mx_paged_attn_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t max_blocks,
                                     int32_t block_size, int32_t chunk_tokens);

int mx_paged_attn_decode(const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint16_t* k, const uint16_t* v,
                         int64_t kv_sblk, int64_t kv_shead, const int32_t* block_tables, int64_t bt_sb,
                         int32_t max_blocks, const int32_t* seq_lens, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                         int32_t block_size, int32_t num_pool_blocks, float scale, uint16_t* out, int64_t o_sb,
                         int64_t o_sh, void* workspace, size_t workspace_bytes, int32_t chunk_tokens, uint32_t flags,
                         void* stream);

/* mx_paged_attn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP-graph capture, serving loops and
 * harnesses that forbid hipMalloc). No counterpart in the reference: its
 * decode path allocates scratch per shape (paged_attention_triton.py:90-115).
 * The split partials live in a static device array of
 * MX_PA_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on
 * until the process ends; shapes whose workspace without the tile plan
 * (mx_paged_attn_workspace_bytes less 1040 bytes per wave) exceeds it are refused
 * with MX_ERR_WORKSPACE, and the plan flags with MX_ERR_INVALID. The call
 * allocates nothing.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (concurrent streams) race, so serialise them. err (nullable) is a
 * caller-owned int32 device word OR-ed with the error bits (bit 0: a block id
 * outside the pool was skipped); without it the bits are dropped. Other
 * arguments, results and status codes are those of mx_paged_attn_decode. */
#define MX_PA_NOALLOC_SCRATCH_BYTES (32u << 20)
int mx_paged_attn_decode_noalloc(const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint16_t* k, const uint16_t* v,
                                 int64_t kv_sblk, int64_t kv_shead, const int32_t* block_tables, int64_t bt_sb,
                                 int32_t max_blocks, const int32_t* seq_lens, int32_t B, int32_t Hq, int32_t Hkv,
                                 int32_t D, int32_t block_size, int32_t num_pool_blocks, float scale, uint16_t* out,
                                 int64_t o_sb, int64_t o_sh, int32_t chunk_tokens, uint32_t flags, int32_t* err,
                                 void* stream);

/* Calibration probe (no reference counterpart; used by bench.py): the K/V reads
 * of mx_paged_attn_decode over the same block tables and lengths, without the
 * math, so its duration is what the gather alone costs on this GPU. mode 0:
 * the decode kernel's own partition and load pattern (default worker count);
 * mode 1: equal ranges of 16-token tiles per workgroup of Hkv waves, wave h
 * reading head h of each tile's block, so a workgroup requests a whole block's
 * Hkv runs (contiguous in the pool) at once. Block size 16, fp16 or bf16 runs
 * (D 64 or 128), Hkv <= 16. Nothing is written except, with negligible odds, a
 * checksum to sink[1] (sink: 2 int32 of device memory). */
int mx_kv_gather_probe(const uint16_t* k, const uint16_t* v, int64_t kv_sblk, int64_t kv_shead,
                       const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks, const int32_t* seq_lens,
                       int32_t B, int32_t Hkv, int32_t D, int32_t block_size, int32_t num_pool_blocks, int32_t mode,
                       int32_t* sink, void* stream);

/* Calibration probe (no reference counterpart; used by bench.py --workload
 * probes): `workgroups` workgroups of `threads` threads (256, 512 or 1024) each
 * read their own contiguous run of bytes_per_wg bytes of src, starting at
 * byte `offset` (runs back to back), with non-temporal 16-byte loads, 4 in
 * flight per thread. The runs must lie inside the src_bytes-byte buffer; sizes
 * and offset are multiples of 16. Nothing is written except, with negligible
 * odds, a checksum to sink[0] (one int32 of device memory). */
int mx_stream_probe(const void* src, int64_t src_bytes, int64_t offset, int64_t bytes_per_wg, int32_t workgroups,
                    int32_t threads, int32_t* sink, void* stream);

/* Calibration probe (no reference counterpart; used by bench.py --workload
 * probes): one launch of `workgroups` workgroups of 256 threads that does
 * nothing (bytes == 0; dst may be NULL) or writes `bytes` bytes of dst, an
 * equal contiguous share per workgroup (bytes a multiple of 16 x workgroups,
 * at most dst_bytes). Its cost inside a HIP graph is the floor under every
 * small launch of the decode step. */
int mx_launch_probe(void* dst, int64_t dst_bytes, int64_t bytes, int32_t workgroups, void* stream);

/* Calibration probe (no reference counterpart; used by bench.py --workload
 * probes): the gather of paged attention without its math. `waves` waves split
 * the n_runs byte offsets (int64 device array) into equal contiguous shares; a
 * wave reads each run of run_bytes (4096 or 8192) bytes from base as coalesced
 * 1 KiB loads, in_flight runs at a time (8192: 1, 2, 3, 4 or 6; 4096: 2 or 4),
 * non-temporal when `streaming` is nonzero (pattern 0). Patterns 1 and 2
 * (8192-byte runs, 2 in flight, streaming) read each run as the paged-attention
 * kernel reads a 16-token K tile of head_dim 128 and its V tile: K as 4 load
 * instructions of 16 rows x 64 bytes, V as 4 of 4 rows x 256 bytes; pattern 2
 * loads the first half of each K line with the default policy, as the kernel
 * does. Pattern 3 stages K through LDS with global->LDS loads of 4 whole token
 * rows each, then reads pattern 1's K operand layout back from LDS; pattern 4
 * also permutes the operand rows so that each V load reads 4 consecutive token
 * rows (1 KiB contiguous). An offset outside [0, base_bytes - run_bytes] reads run 0 instead
 * (offsets round down to 16 bytes), so no list reads outside the buffer.
 * Nothing is written except, with negligible odds, a checksum to sink[0]. */
int mx_run_gather_probe(const void* base, int64_t base_bytes, const int64_t* offsets, int64_t n_runs,
                        int32_t run_bytes, int32_t waves, int32_t in_flight, int32_t streaming, int32_t pattern,
                        int32_t* sink, void* stream);

/* Calibration probe (no reference counterpart; used by bench.py --workload
 * probes): what handing data between the workgroups of one launch costs
 * against a launch boundary. `workgroups` workgroups of 256 threads each write
 * an 8 KiB fp32 partial to part (float i of workgroup w: (31 w + i) & 1023);
 * the partials of each group of `group` consecutive workgroups are summed in
 * workgroup order into out[w / group] (2048 floats). Mode 0: the partials
 * only (out untouched); 1: the partials, then a second launch that sums each
 * group; 2: the group's last workgroup to take a ticket sums them, behind
 * agent-scope release/acquire fences; 3: the same with sequentially
 * consistent fences; 4: the same without fences, the partials written and
 * read device-coherent. tickets (one int32 per group, modes 2-4) must be zero
 * before the first call; each call leaves them zero. part and out 16-byte
 * aligned. */
int mx_handoff_probe(float* part, int64_t part_bytes, float* out, int64_t out_bytes, int32_t* tickets,
                     int64_t tickets_bytes, int32_t workgroups, int32_t group, int32_t mode, void* stream);

/* Calibration probe (no reference counterpart; used by bench.py --workload
 * probes): `workgroups` workgroups of 512 threads, all resident at once (else
 * MX_ERR_UNSUPPORTED), pass `rounds` grid barriers. Mode 0: one counter,
 * polled by thread 0; 1: one flag per workgroup, wave 0 polls them all; 2: 8
 * counters, polled by 8 threads; 3: as 2, with 1 KiB per workgroup handed to
 * the next workgroup each round through device-coherent stores and loads
 * (hand: 2 KiB per workgroup, 16-byte aligned); 4: as 3 with plain stores and
 * loads behind agent-scope release/acquire fences. sync (16 + workgroups int32)
 * must be zero before the first call; each call leaves it zero. Waits are
 * bounded: a wait that times out sets err bit 1 (the launch still ends); a
 * hand-off that reads a wrong value sets bit 2. */
int mx_barrier_probe(int32_t* sync, int64_t sync_bytes, int32_t* hand, int64_t hand_bytes, int32_t workgroups,
                     int32_t rounds, int32_t mode, int32_t* err, void* stream);

/* Calibration probe (no reference counterpart; used by bench.py --workload
 * probes): a chain of phases, each streaming bytes_per_wg distinct bytes per
 * workgroup of src (phase p, workgroup w: the run at (p x workgroups + w) x
 * bytes_per_wg) and handing 1 KiB per workgroup to the next phase (workgroup w
 * reads what w + 1 wrote; phase p writes p + 1, a wrong value sets err bit 2).
 * persistent == 0 runs phases [phase0, phase0 + phases) with plain hand-off
 * stores and loads: one phase per call is the graph of kernels. persistent !=
 * 0 runs phases [0, phases) in one launch of resident workgroups (else
 * MX_ERR_UNSUPPORTED): each phase issues its first loads (up to 128 KiB per
 * workgroup), waits at an 8-counter grid barrier (sync: 9 int32, zero before
 * the first call, left zero), and hands over through device-coherent stores
 * and loads; a wait that times out sets err bit 1. hand: 2 KiB per workgroup, 16-byte aligned. Nothing
 * else is written except, with negligible odds, a checksum to sink[0]. */
int mx_chain_probe(const void* src, int64_t src_bytes, int64_t bytes_per_wg, int32_t workgroups, int32_t phase0,
                   int32_t phases, int32_t persistent, int32_t* sync, int64_t sync_bytes, int32_t* hand,
                   int64_t hand_bytes, int32_t* err, int32_t* sink, void* stream);

/* Byte offset of the int32 error word inside a paged-attention workspace
 * (nonzero after a call that met an out-of-range block id). Reading it needs a
 * device-to-host copy by the caller; clearing it is the caller's choice. */
size_t mx_paged_attn_error_offset(int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t max_blocks,
                                  int32_t block_size, int32_t chunk_tokens);

/* ----------------------------------------------------------------------------
 * Decode-step glue.
 *
 * The element-wise work of a decoder layer around the linears and the
 * attention call. In the reference these are torch ops inside the HF decoder
 * layer (transformers' RMSNorm, apply_rotary_pos_emb and SwiGLU MLP, a
 * third-party library reached from the batched decode forward,
 * runtime/phase2/worker_server.py:771-775) and the KV scatter of
 * GpuKVBlockPool.write_tokens_batch (runtime/phase2/paged_kv_kernel.py:176-227),
 * called by BlockPagedBatchLayer.update (runtime/phase2/paged_kv_cache.py:121-157).
 * Out-of-range slots are skipped, never written, and OR-ed into *err when err
 * is not NULL (bit 0: logical block past max_blocks or physical id outside
 * [0, num_pool_blocks); bit 1: position outside the rotary table).
 * ------------------------------------------------------------------------- */

/* Scatter new K/V states [B, Hkv, T, D] (strides new_sb, new_sh, new_st; D
 * contiguous) into per-layer pool views [num_blocks, Hkv, block_size, D]
 * (strides kv_sblk, kv_shead, D, 1): token t of row b goes to position
 * start_pos[b] + t, i.e. block block_tables[b, pos / block_size] at offset
 * pos % block_size. Replaces write_tokens_batch (paged_kv_kernel.py:176-227;
 * the reference loops over tokens on the host and checks bounds with host
 * syncs, :217-227). D % 8 == 0; rows 16-byte aligned. used_blocks (nullable,
 * uint8 [num_pool_blocks]) gets 1 at every physical block a token was written
 * to: the block-usage accounting of the reference's _touch_blocks (:229-231)
 * kept on the device, read only when the caller asks. */
int mx_kv_append(const uint16_t* k_new, const uint16_t* v_new, int64_t new_sb, int64_t new_sh, int64_t new_st,
                 int32_t B, int32_t T, int32_t Hkv, int32_t D, const int32_t* block_tables, int64_t bt_sb,
                 int32_t max_blocks, const int32_t* start_pos, uint16_t* k_pool, uint16_t* v_pool, int64_t kv_sblk,
                 int64_t kv_shead, int32_t block_size, int32_t num_pool_blocks, int32_t* err, uint8_t* used_blocks,
                 void* stream);

/* From one fused QKV projection row per sequence (fp16 [B, (Hq + 2*Hkv) * D],
 * row stride qkv_stride; heads in the order q, k, v): rotate q and k with
 * rotate-half RoPE at position positions[b] (pairs i, i + D/2 use
 * rope[pos][i] = (cos, sin), an fp32 table of max_pos rows), write q to
 * q_out [B, Hq * D] (row stride q_stride) and k, v to the pool slot of
 * position positions[b] (as mx_kv_append). Replaces HF's
 * apply_rotary_pos_emb (transformers, reached from worker_server.py:771-775)
 * followed by BlockPagedBatchLayer.update's write (paged_kv_cache.py:121-157).
 * A position outside the table writes q = 0 and no K/V. lens_out (optional,
 * int32 [B]) receives positions[b] + 1, the KV length the attention call of
 * this token reads (seq_lens in paged_attention_triton.py:43-50). used_blocks
 * (nullable) is marked as by mx_kv_append. */
int mx_qkv_rope_append(const uint16_t* qkv, int64_t qkv_stride, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                       const float* rope, int32_t max_pos, const int32_t* positions, uint16_t* q_out,
                       int64_t q_stride, uint16_t* k_pool, uint16_t* v_pool, int64_t kv_sblk, int64_t kv_shead,
                       const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks, int32_t block_size,
                       int32_t num_pool_blocks, int32_t* err, int32_t* lens_out, uint8_t* used_blocks,
                       void* stream);

/* mx_qkv_rope_append with the QKV projection given as split-K partials
 * (fp32 [splits][B][(Hq + 2*Hkv) * D], from mx_w8a16_linear_partials): each
 * element is fp16(sum over splits + bias), the value mx_w8a16_linear would
 * have written, then rotated and appended as above. bias may be NULL;
 * partials and bias need 16-byte alignment. */
int mx_qkv_rope_append_splits(const float* partials, int32_t splits, const uint16_t* bias, int32_t B, int32_t Hq,
                              int32_t Hkv, int32_t D, const float* rope, int32_t max_pos, const int32_t* positions,
                              uint16_t* q_out, int64_t q_stride, uint16_t* k_pool, uint16_t* v_pool, int64_t kv_sblk,
                              int64_t kv_shead, const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks,
                              int32_t block_size, int32_t num_pool_blocks, int32_t* err, int32_t* lens_out,
                              uint8_t* used_blocks, void* stream);

/* The QKV projection and mx_qkv_rope_append_splits in one launch, for the
 * decode step's first two kernels per layer: q = the rotated q heads of
 * x[M, K] W^T (+ bias) (W the packed fused-QKV weight, N = (Hq + 2*Hkv) * D
 * rows in the order q, k, v), k rotated and v appended at position
 * positions[m], with everything else (q_out layout, pool slots, errors,
 * lens_out, used_blocks) as in mx_qkv_rope_append. The result is bit for bit that of
 * mx_w8a16_linear_partials followed by mx_qkv_rope_append_splits whenever
 * mx_w8a16_splits(M, N, K) == 8 (the decode step's qkv at 5 <= M <= 32 on the
 * Llama-3-8B shape): each of the kernel's 8 waves accumulates one of those
 * split ranges. Replaces the HF q/k/v projections, apply_rotary_pos_emb and
 * BlockPagedBatchLayer.update's write (worker_server.py:771-775,
 * paged_kv_cache.py:121-157). 1 <= M <= 32; D in {64, 128}; K % 64 == 0;
 * M > 32 returns MX_ERR_UNSUPPORTED (use the two-launch path). */
int mx_w8a16_qkv_rope_append(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride, const uint8_t* packed,
                             const uint16_t* scale, const uint16_t* bias, int32_t Hq, int32_t Hkv, int32_t D,
                             const float* rope, int32_t max_pos, const int32_t* positions, uint16_t* q_out,
                             int64_t q_stride, uint16_t* k_pool, uint16_t* v_pool, int64_t kv_sblk, int64_t kv_shead,
                             const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks, int32_t block_size,
                             int32_t num_pool_blocks, int32_t* err, int32_t* lens_out, uint8_t* used_blocks,
                             void* stream);

/* h = residual ? fp16(x + residual) : x;  residual_out (if not NULL) = h;
 * out = fp16(fp16(h * rsqrt(mean(h^2) + eps)) * weight), per row of H
 * (H % 8 == 0, H <= 16384). The decoder layer's residual add and the
 * following RMSNorm (transformers' Qwen2/Llama RMSNorm, reached from
 * worker_server.py:771-775) in one pass. x_rows (optional, int64 [M]) gathers
 * row m of x from row x_rows[m] (the embedding lookup of a step's tokens); x
 * then holds x_count rows and an index outside [0, x_count) reads a zero row.
 * out may alias x and residual_out may alias residual; out must not alias
 * residual_out. */
int mx_add_rmsnorm(const uint16_t* x, int64_t x_stride, const int64_t* x_rows, int64_t x_count,
                   const uint16_t* residual, int64_t r_stride, const uint16_t* weight, int32_t M, int32_t H,
                   float eps, uint16_t* out, int64_t out_stride, uint16_t* residual_out, int64_t ro_stride,
                   void* stream);

/* mx_add_rmsnorm with x given as the split-K partials of the linear that
 * produced it (fp32 [splits][M][H] from mx_w8a16_linear_partials): x =
 * fp16(sum over splits + bias) as mx_w8a16_linear would have written it; the
 * rest is mx_add_rmsnorm. bias may be NULL. */
int mx_add_rmsnorm_splits(const float* partials, int32_t splits, const uint16_t* bias, const uint16_t* residual,
                          int64_t r_stride, const uint16_t* weight, int32_t M, int32_t H, float eps, uint16_t* out,
                          int64_t out_stride, uint16_t* residual_out, int64_t ro_stride, void* stream);

/* out[m] = index of the largest of logits[m, 0..N) (fp16, row stride
 * `stride`), the first on ties, NaN above any number: the greedy argmax of the
 * decode step (worker_server.py:786, torch argmax over the last logits).
 * seq_lens (optional, int32 [M]) is incremented by one per row, advancing the
 * KV lengths past the token just decoded. */
int mx_argmax_rows(const uint16_t* logits, int64_t stride, int32_t M, int32_t N, int64_t* out, int32_t* seq_lens,
                   void* stream);

/* mx_argmax_rows with each row cut into 4096-logit chunks reduced by separate
 * workgroups (two launches on `stream`), for rows too long for one CU to read
 * fast: the same results (first index on ties, -0 == +0, the first NaN above
 * any number). workspace: at least mx_argmax_workspace_bytes(M, N) bytes,
 * 8-byte aligned, not shared by concurrent calls; it needs no initialisation.
 * M <= 65535. Same reference counterpart as mx_argmax_rows
 * (worker_server.py:786). */
size_t mx_argmax_workspace_bytes(int32_t M, int32_t N);
int mx_argmax_rows_split(const uint16_t* logits, int64_t stride, int32_t M, int32_t N, int64_t* out,
                         int32_t* seq_lens, void* workspace, size_t workspace_bytes, void* stream);

/* SwiGLU of the interleaved gate||up projection used by mx_w8a16_gateup_swiglu
 * (rows 16t + [0, 8) gate channels 8t + [0, 8), rows 16t + [8, 16) the matching
 * up channels): out[m, 8t + e] = fp16(fp16(silu(g)) * u), with g and u rounded
 * to fp16 as that projection's output is. Input is either its fp16 output rows
 * (gate_up, [M, 2I], row stride gu_stride; partials NULL) or its split-K
 * partials (partials [splits][M][2I] from mx_w8a16_linear_partials plus bias,
 * summed bias-first in split order exactly as mx_w8a16_linear's reduce;
 * gate_up NULL). For the shapes mx_w8a16_gateup_swiglu does not take (M <= 4,
 * or gate||up split over K): HF MLP act_fn(gate_proj(x)) * up_proj(x),
 * reached from worker_server.py:771-775. I % 8 == 0. */
int mx_swiglu_interleaved(const uint16_t* gate_up, int64_t gu_stride, const float* partials, int32_t splits,
                          const uint16_t* bias, int32_t M, int32_t I, uint16_t* out, int64_t out_stride,
                          void* stream);

/* out[m, i] = fp16(fp16(silu(gate_up[m, i])) * gate_up[m, I + i]) for i < I
 * (I % 8 == 0): the SwiGLU product between the fused gate||up projection and
 * the down projection (transformers' MLP act_fn(gate_proj(x)) * up_proj(x),
 * reached from worker_server.py:771-775). */
int mx_silu_mul(const uint16_t* gate_up, int64_t gu_stride, int32_t M, int32_t I, uint16_t* out,
                int64_t out_stride, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MXDECODE_H */
