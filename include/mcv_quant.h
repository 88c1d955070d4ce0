/*
 * mcv_quant.h -- C-ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * This is the boundary below the C++ operator surface (namespace minicpmv, see
 * minicpm-v-4.6-orangepi_amd/cpp/include/minicpmv/).  In the reference that
 * boundary is the aclnn two-phase ABI generated from each custom operator's
 * OpDef, e.g. aclnnMatmulW4a16CustomGetWorkspaceSize + aclnnMatmulW4a16Custom
 * (src/csrc/lib/ops.cpp:1087-1094, OpDef src/csrc/custom_ops/op_host/
 * matmul_w4a16_custom.cpp:47-75).  Here each operator is one plain function.
 *
 * Conventions
 *   - Only plain pointers, sizes and enums cross the boundary.  Pointers named
 *     *_dev are device (HBM) pointers; *_host are host pointers.  fp16 data is
 *     passed as raw IEEE binary16 bits (uint16_t / void*).
 *   - Device entry points are stream-ordered and asynchronous on `stream`
 *     (a hipStream_t; NULL means the legacy default stream).  They never
 *     allocate or free caller memory and never synchronise, except where noted.
 *   - Every entry point returns MCV_OK (0) or an MCV_ERR_* code; the message of
 *     the last failure on the calling thread is returned by mcv_last_error().
 *   - Shapes are validated on the host before any launch; a bad shape is an
 *     error return, never a kernel launch.
 *
 * W4A16 weight layout on the device ("slab-64", MCV_W4_LAYOUT_SLAB64)
 *   A K x N int4 weight (K % 128 == 0, any N >= 1) is cut into slabs of 64
 *   output columns (Npad = 64 * ceil(N / 64); padding columns are zero) and
 *   chunks of 32 k.  One chunk of one slab is 1 KiB: 64 lanes x 16 bytes,
 *   lane l holding column 64*slab + l, so a wave's 128-bit loads are one
 *   contiguous 1 KiB line.  Byte offset of (slab, chunk c, lane l) =
 *   ((slab * (K/32) + c) * 64 + l) * 16; within those 16 bytes word w
 *   (little-endian uint32) holds k = 32c + 8w + order[s] in nibble s
 *   (bits 4s..4s+3), order = {0,2,4,6,1,3,5,7}.
 *   Scales: fp16 [K/128][Npad] (zero for padding columns).
 *   Zeros: uint32 [K/128][Npad/8], nibble s of word j holding column 8j + s.
 *   Effective zero = nibble + zero_bias (0 for AWQ/synthetic, 1 for GPTQ v1).
 *   Dequantised value w[k][n] = (q - (z + zero_bias)) * s[k/128][n].
 *
 * W8A8 weight layout MCV_W8_TILED
 *   A K x N int8 weight is padded with zeros to Np = 64 * ceil(N / 64)
 *   columns and Kp = 128 * ceil(K / 128) rows and stored as 1 KiB operand
 *   lines of 32 columns x 32 k: byte offset of w[k][n] =
 *     ((((n / 64) * (Kp / 32) + k / 32) * 2 + (n % 64) / 32) * 64 + l) * 16 + (k % 16),
 *   l = (n % 32) + 32 * ((k % 32) / 16): the operand order of
 *   v_mfma_i32_32x32x32_i8, so a wave loads each operand with one coalesced
 *   128-bit load.  Size: mcv_w8a8_tiled_bytes(K, N) = Np * Kp.
 */
#ifndef MCV_QUANT_H
#define MCV_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mcv_stream_t; /* hipStream_t */

enum mcv_status {
    MCV_OK = 0,
    MCV_ERR_INVALID_ARG = 1, /* null pointer, bad enum, bad size */
    MCV_ERR_SHAPE = 2,       /* shape constraint violated */
    MCV_ERR_HIP = 3,         /* HIP runtime error (launch, device query) */
    MCV_ERR_UNSUPPORTED = 4, /* input format the library cannot represent */
    MCV_ERR_NO_DEVICE = 5    /* no usable gfx950 device / kernels not loadable */
};

enum mcv_dtype { MCV_F32 = 0, MCV_F16 = 1 };
enum mcv_w8_layout {
    MCV_W8_KN = 0,    /* [K][N] row-major, the reference's layout */
    MCV_W8_NK = 1,    /* [N][K] row-major */
    MCV_W8_TILED = 2  /* MFMA operand tiles, see below */
};

#define MCV_W4_GROUP 128
#define MCV_W4_LAYOUT_SLAB64 1

/* Message of the last failed call on this thread ("" if none).  Replaces the
 * std::runtime_error text of check_acl (src/csrc/include/minicpmv/acl_context.h:11-15). */
const char* mcv_last_error(void);
/* Library version string. */
const char* mcv_version(void);

/* ---------------------------------------------------------------- sizes -- */
/* Byte sizes of the slab-64 packed tensors for a K x N weight (0 on bad shape). */
int64_t mcv_w4a16_packed_weight_bytes(int64_t K, int64_t N);
int64_t mcv_w4a16_packed_scale_bytes(int64_t K, int64_t N);
int64_t mcv_w4a16_packed_zero_bytes(int64_t K, int64_t N);

/* ---------------------------------------------------- host-side packers -- */
/* Replaces unpack_awq_weight + pack_w4a16_weight
 * (src/csrc/lib/quantized_weight.cpp:122-160, 48-73): AutoAWQ gemm tensors
 * (qweight int32 [K][N/8], qzeros int32 [K/128][N/8], scales fp16 [K/128][N])
 * to slab-64.  Nibbles are re-laid, never widened to int8.  zero_bias = 0.
 * Output buffers are host memory of the mcv_w4a16_packed_*_bytes sizes. */
int mcv_w4a16_pack_awq(const int32_t* qweight_host, const int32_t* qzeros_host,
                       const uint16_t* scales_host, int64_t K, int64_t N,
                       void* qw_host, uint16_t* scales_out_host, uint32_t* zeros_out_host);

/* Replaces unpack_gptq_weight + pack_w4a16_weight
 * (src/csrc/lib/quantized_weight.cpp:75-120, 48-73): GPTQ v1 tensors (qweight
 * int32 [K/8][N], qzeros int32 [G][N/8], g_idx int32 [K] or NULL, scales fp16
 * [G][N]) to slab-64 with zero_bias = 1 (GPTQ stores zero - 1, :112).  With
 * an act-order g_idx (:98-117) row k's zero comes from group g_idx[k] while
 * the scale stays that of group k/128, as in the reference; the int8 values
 * q - zero are kept exact by re-basing each (k/128 group, column) on one
 * common zero (unchanged nibbles when the rows' zeros agree, as in every
 * sym=True checkpoint).  MCV_ERR_SHAPE for g_idx outside [0, G);
 * MCV_ERR_UNSUPPORTED when one group's values span more than 16 levels (the
 * loaders then keep the weight dense: mcv_w4a16_dequant_gptq_host). */
int mcv_w4a16_pack_gptq(const int32_t* qweight_host, const int32_t* qzeros_host,
                        const int32_t* g_idx_host, const uint16_t* scales_host,
                        int64_t K, int64_t N, int64_t groups,
                        void* qw_host, uint16_t* scales_out_host, uint32_t* zeros_out_host);

/* When mcv_w4a16_pack_gptq returns MCV_ERR_UNSUPPORTED (an act-order block's
 * values span more than 16 levels): the dense fp16 weight w_kn_host [K][N],
 * element (k, n) = RNE((q - zero[g_idx[k]]) * scale[k/128][n]), the
 * reference's values (quantized_weight.cpp:98-117 with the kernel's scale by
 * position), for a plain fp16 GEMM.  Same tensors and errors as
 * mcv_w4a16_pack_gptq; g_idx may be NULL. */
int mcv_w4a16_dequant_gptq_host(const int32_t* qweight_host, const int32_t* qzeros_host,
                                const int32_t* g_idx_host, const uint16_t* scales_host, int64_t K,
                                int64_t N, int64_t groups, uint16_t* w_kn_host);

/* Build-defined synthetic int4 quantiser (the reference has none; it only
 * unpacks AutoAWQ/GPTQ checkpoints).  Per (group g, column n) over the 128
 * fp16 values w of the group: s = fp16_rne(max(max(w) - min(w), 1e-5) / 15),
 * z = clamp(rne(-min(w) / s), 0, 15), q = clamp(rne(w / s) + z, 0, 15).
 * Output is AutoAWQ gemm packing (qweight int32 [K][N/8], qzeros int32
 * [K/128][N/8], scales fp16 [K/128][N]), readable by the reference's
 * unpack_awq_weight (src/csrc/lib/quantized_weight.cpp:122-160) and by
 * mcv_w4a16_pack_awq.  w_kn_host is fp16 [K][N], K % 128 == 0, N % 8 == 0.
 * Runs on up to `nthreads` host threads (<= 0: all hardware threads). */
int mcv_w4a16_quantize_host(const uint16_t* w_kn_host, int64_t K, int64_t N, int32_t* qweight_host,
                            int32_t* qzeros_host, uint16_t* scales_host, int nthreads);

/* The same quantiser fed from an [N_src][K] (out, in) fp16 or bf16 tensor --
 * the tied embedding [vocab, hidden] that the lm_head reuses as its
 * projection -- with the output padded to N columns (N % 8 == 0, N >= N_src):
 * columns from N_src on are zero weights (q = z = 0).  Outputs as above,
 * [K][N/8] / [K/128][N/8] / [K/128][N].  Bit-identical to
 * mcv_w4a16_quantize_host on the transposed, zero-padded [K][N] (bf16 source
 * values converted as mcv_w8a8_quantize_weight_nk_host converts them). */
int mcv_w4a16_quantize_nk_host(const uint16_t* w_nk_host, int src_dtype, int64_t K, int64_t N_src, int64_t N,
                               int32_t* qweight_host, int32_t* qzeros_host, uint16_t* scales_host, int nthreads);

/* Inverse of the packers, for round trips and inspection: writes the nibble q
 * ([K][N] uint8, may be NULL), the effective zero z + zero_bias ([K/128][N]
 * uint8, may be NULL) and the unpadded scales ([K/128][N] fp16, may be NULL). */
int mcv_w4a16_unpack_host(const void* qw_host, const uint16_t* scales_host,
                          const uint32_t* zeros_host, int zero_bias, int64_t K, int64_t N,
                          uint8_t* q_kn_host, uint8_t* zeff_gn_host, uint16_t* scales_gn_host);

/* ------------------------------------------------------ W4A16 on device -- */
/* out[M][N] fp16 = x[M][K] fp16 . dequant(W) with fp32 accumulation.
 * Replaces matmul_w4a16 / aclnnMatmulW4a16Custom (src/csrc/lib/ops.cpp:1030-1095,
 * kernel src/csrc/custom_ops/op_kernel/matmul_w4a16_custom.cpp:157-168), which
 * accepts M = 1 only; any M >= 1 is accepted here.  Small M runs the streaming
 * GEMV kernel, larger M the LDS-dequant fp16 MFMA GEMM, unsplit (without a
 * workspace it never splits K; mcv_w4a16_gemm_ws may). */
int mcv_w4a16_gemm(const void* x_dev, int64_t M, int64_t K, int64_t N,
                   const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                   int zero_bias, void* out_dev, mcv_stream_t stream);

/* mcv_w4a16_gemm with a caller-owned device workspace (no counterpart in the
 * reference, whose matmul_w4a16 is M = 1 only): where the MFMA tile grid is
 * small (few rows, long K) the GEMM splits K across workgroups inside the
 * same launch -- each writes an fp32 partial tile, the last of a tile adds
 * them in split order and rounds to fp16 (deterministic; the sum order
 * differs from the unsplit kernel's, within the same fp32 accumulation
 * tolerance).  The workspace must be 256-byte aligned, hold
 * mcv_w4a16_gemm_workspace_bytes(M, K, N) bytes (else the call runs
 * unsplit) and be zero-filled once before its first use: its first 4 KiB hold
 * the tiles' arrival counters, which every call leaves zero, so one workspace
 * serves calls of every shape.  Calls that share a workspace must be ordered
 * (one stream). */
int mcv_w4a16_gemm_ws(const void* x_dev, int64_t M, int64_t K, int64_t N,
                      const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                      int zero_bias, void* out_dev, void* workspace_dev, int64_t workspace_bytes,
                      mcv_stream_t stream);

/* Workspace bytes mcv_w4a16_gemm_ws uses for this shape (0: it does not split
 * K, and any workspace, NULL included, is ignored). */
int64_t mcv_w4a16_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N);

/* The kernel (and configuration) mcv_w4a16_gemm (with_workspace = 0) or
 * mcv_w4a16_gemm_ws (1) launches for M x K x N, as text, for labels in
 * reports; valid until the next call on this thread.  No reference
 * counterpart. */
const char* mcv_w4a16_gemm_kernel_name(int64_t M, int64_t K, int64_t N, int with_workspace);

/* The half-slab GEMM with an explicit configuration (what mcv_w4a16_gemm_ws
 * picks by shape; exposed so every configuration can be tested and timed):
 * tile tm x 32 * waves (tm in {32, 64, 128}, waves in {2, 4, 8}), `stages`
 * copy stages in flight of `groups_per_stage` quantisation groups (128 k)
 * each, `k_parts` waves per half-slab (1, or 2 with groups_per_stage 2:
 * each takes one group of every stage), `weights_in_registers` 1 to load
 * each wave's packed weights, zeros and scales straight into registers (the
 * stage buffers in LDS then hold x rows only), `tile_order` the order in
 * which the XCDs take the tiles (0 as the dispatch: down the tile columns when
 * x has fewer bytes than the packed weights, else as 3; 1 along the rows; 2
 * down the columns; 3 down the columns of groups of tile rows sized so that
 * each XCD's run of tiles spans about as many x bytes as weight bytes), K
 * split `splits` ways across
 * workgroups (groups_per_stage divides K / 128, splits at most
 * K / 128 / groups_per_stage; split p takes stages [p U / S, (p+1) U / S) of
 * the U = K / 128 / groups_per_stage), the partial tiles added inside the same launch by the
 * last workgroup of each tile, in split order (deterministic).  Splits > 1
 * need a 256-byte aligned workspace of mcv_w4a16_gemm_sk_workspace_bytes
 * bytes, zero-filled once before its first use: its first 4 KiB hold the
 * tile arrival counters (at most 1024 tiles per split call), which every
 * call leaves zero, so one workspace serves calls of every shape.
 * MCV_ERR_INVALID_ARG for a configuration that is not built.
 * No reference counterpart (the reference has no quantised M > 1 path). */
int64_t mcv_w4a16_gemm_sk_workspace_bytes(int64_t M, int64_t N, int tm, int waves, int splits);
int mcv_w4a16_gemm_sk(const void* x_dev, int64_t M, int64_t K, int64_t N,
                      const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                      int zero_bias, void* out_dev, int tm, int waves, int stages,
                      int groups_per_stage, int k_parts, int weights_in_registers, int tile_order,
                      int splits, void* workspace_dev, int64_t workspace_bytes, mcv_stream_t stream);

/* The two kernels behind mcv_w4a16_gemm, callable directly (same contract). */
int mcv_w4a16_gemv(const void* x_dev, int64_t M, int64_t K, int64_t N,
                   const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                   int zero_bias, void* out_dev, mcv_stream_t stream);
int mcv_w4a16_gemm_mfma(const void* x_dev, int64_t M, int64_t K, int64_t N,
                        const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                        int zero_bias, void* out_dev, mcv_stream_t stream);

/* Decode MLP front half in one launch: act[M][N] = silu(x . Wgate) * (x . Wup)
 * with gate and up rounded to fp16 first, exactly as two mcv_w4a16_gemv calls
 * followed by mcv_silu_mul produce it (bit-identical).  Both weights are K x N
 * slab-64.  Replaces the gate matmul + up matmul + silu_mul sequence of the
 * decoder layers' MLP (src/csrc/lib/decoder_layer.cpp:1029-1046, silu_mul
 * src/csrc/lib/ops.cpp:437-456).  Meant for decode-sized M (GEMV kernel). */
int mcv_w4a16_gate_up_silu(const void* x_dev, int64_t M, int64_t K, int64_t N,
                           const void* qw_gate_dev, const void* scales_gate_dev, const void* zeros_gate_dev,
                           int zero_bias_gate, const void* qw_up_dev, const void* scales_up_dev,
                           const void* zeros_up_dev, int zero_bias_up, void* act_dev, mcv_stream_t stream);

/* The whole decode MLP block, M = 1, in one launch:
 *   out[H] = (silu(x . Wgate) * (x . Wup)) . Wdown
 * gate/up H x I and down I x H, all slab-64; bit-identical to
 * mcv_w4a16_gate_up_silu followed by mcv_w4a16_gemm on its output.  Replaces
 * the decoder layers' MLP sequence (src/csrc/lib/decoder_layer.cpp:1029-1046:
 * gate and up matmul_w4a16, silu_mul, down matmul_w4a16).  H and I are
 * multiples of 128 with I <= 4096 (at most two quantisation groups of the
 * down projection per wave slot), and the launch must fit on the device all
 * at once (MCV_ERR_SHAPE otherwise: use the two-launch sequence).  The act row
 * and the down projection's partial sums pass between workgroups inside the
 * kernel through `workspace_dev` (per-workgroup call counters and call-tagged
 * words): mcv_w4a16_mlp_workspace_bytes(H, I) bytes, 256-byte aligned,
 * zero-filled once before the first call; one workspace serves one (H, I)
 * shape, and calls sharing it must not overlap.  Every wait is bounded: if a
 * wait for another workgroup's words gives up (after ~0.3 s -- e.g. another
 * stream's kernels kept part of the grid from being resident), the u32 at
 * byte 0 of the workspace becomes non-zero, and so does `*status` when status
 * is not NULL, and the output of that call is undefined.  status may point to
 * host-mapped pinned memory (hipHostMalloc + hipHostGetDevicePointer), where
 * the host sees a give-up without synchronising.  After a give-up the
 * workspace must be zero-filled again before the next call. */
int64_t mcv_w4a16_mlp_workspace_bytes(int64_t H, int64_t I);
int mcv_w4a16_mlp(const void* x_dev, int64_t H, int64_t I,
                  const void* qw_gate_dev, const void* scales_gate_dev, const void* zeros_gate_dev, int zero_bias_gate,
                  const void* qw_up_dev, const void* scales_up_dev, const void* zeros_up_dev, int zero_bias_up,
                  const void* qw_down_dev, const void* scales_down_dev, const void* zeros_down_dev,
                  int zero_bias_down, void* out_dev, void* workspace_dev, uint32_t* status,
                  mcv_stream_t stream);

/* Materialise dequantised weights: w_f16_kn [K][N] = fp16 RNE((q - z) * s)
 * and/or w8_kn [K][N] = q - z (int8), either may be NULL.  The int8 form is
 * the reference's unpacked w_int8 (src/csrc/lib/quantized_weight.cpp:155). */
int mcv_w4a16_dequant(const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                      int zero_bias, int64_t K, int64_t N,
                      void* w_f16_kn_dev, int8_t* w8_kn_dev, mcv_stream_t stream);

/* The reference's own W4A16 device format: int8 (q - z) tile-packed by
 * pack_w4a16_weight (src/csrc/lib/quantized_weight.cpp:41-73) into
 * [(K/128)*8*tilesPerBlock*128][tile_len], fp16 scales [K/128][N], M = 1.
 * Same validation as src/csrc/lib/ops.cpp:1037-1079. */
int mcv_w4a16_gemv_tiled_i8(const void* x_dev, int64_t K, int64_t N, int64_t tile_len,
                            int64_t packed_rows, const int8_t* w_dev, const void* scales_dev,
                            void* out_dev, mcv_stream_t stream);

/* One W4A16 projection of a shared activation row, for mcv_w4a16_gemv_multi. */
typedef struct mcv_w4a16_part {
    const void* qw_dev;        /* slab-64 nibbles of a K x N weight */
    const void* scales_dev;
    const void* zeros_dev;
    int zero_bias;
    int64_t N;
    void* out_dev;             /* fp16 [M][N] */
} mcv_w4a16_part;

/* Up to four projections of the same x [M][K] in one launch: the decode
 * step's q/k/v (src/csrc/lib/decoder_layer.cpp:970-972) or qkv and z
 * (:1108-1110), which the reference dispatches one matmul_decode_dispatch at a
 * time.  Each part's output equals mcv_w4a16_gemv on that weight when both
 * split K the same way (every K = 1024 decode shape). */
int mcv_w4a16_gemv_multi(const void* x_dev, int64_t M, int64_t K, const mcv_w4a16_part* parts, int n_parts,
                         mcv_stream_t stream);

/* Workspace for mcv_w4a16_lm_head_argmax over V columns (0 < V < 2^24):
 * device memory of this many bytes, 128-byte aligned, zero-filled once before
 * its first use.  It holds a generation word and the call-tagged key words of
 * the fused argmax, which every call keeps consistent: a workspace sized for
 * the largest V serves every smaller V too, eager calls and HIP-graph replays
 * alike, but calls sharing it must not overlap.  The u32 at byte 0 turns
 * non-zero if the wait for the keys ever gave up (~40 ms); that call's token
 * is then -1, and later calls need no reset.  Returns 0 for an unsupported V. */
int64_t mcv_lm_head_workspace_bytes(int64_t V);

/* Slabs of 64 columns per workgroup that the lm_head entry points launch for
 * V columns (1, 2, 4, 8 or 16; a function of V alone), or 0 for an
 * unsupported V.  A query for labels and tuning reports; no reference
 * counterpart (the reference's lm_head runs 16 chunk matmuls). */
int64_t mcv_lm_head_slabs_per_workgroup(int64_t V);

/* Greedy lm_head over a W4A16 weight: logits[v] = x . W[:, v] (fp16 RNE of the
 * fp32 sum) for v < V, and token = the first index of the maximum logit, with
 * fp16 subnormals compared as zero and NaN never winning (language_model.cpp:
 * 444-479).  x is [1][K]; the weight is K x N as packed (N >= V; columns from
 * V on are ignored, like the reference's clipped chunk tails, :472).
 * logits_dev may be NULL.  token_dev receives an int64 on the device.
 * Replaces the 16 chunk matmuls + 16 D2H copies + host scan of lm_head_greedy
 * (src/csrc/lib/language_model.cpp:412-482) with one kernel: each workgroup
 * of the GEMV publishes its best (value, index) as one call-tagged word in the
 * workspace, and the grid's last workgroup waits until all carry this call's
 * tag, takes the maximum and writes the token.  If that bounded wait gives up
 * the token is -1, the workspace's give-up word is set and so is `*status`
 * (may be NULL; host-mapped pinned memory works, as for mcv_w4a16_mlp). */
int mcv_w4a16_lm_head_argmax(const void* x_dev, int64_t K, int64_t N, int64_t V,
                             const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                             int zero_bias, void* logits_dev, int64_t* token_dev,
                             void* workspace_dev, uint32_t* status, mcv_stream_t stream);

/* The device-token lm_head above for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Identical arguments
 * and results to mcv_w4a16_lm_head_argmax, minus the workspace: the
 * workspace lives in a library-owned array in device memory, one per GPU,
 * held until the process ends, for V <= mcv_lm_head_noalloc_max_vocab()
 * (2^20; larger V is MCV_ERR_SHAPE).  The call allocates nothing and
 * launches only the lm_head kernel, so it may be captured into a HIP graph;
 * captured replays and eager calls at other V may interleave, because the
 * array's state lives in device memory and is valid for every V.  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race and give undefined tokens.  A bounded
 * wait that gives up shows as token -1 and *status (when not NULL); the next
 * call needs no reset. */
int64_t mcv_lm_head_noalloc_max_vocab(void);
/* Test hook, no use in production: while on, the device-token lm_head's
 * poller (mcv_w4a16_lm_head_argmax and _noalloc) expects a tag no key carries,
 * so its bounded wait gives up (token -1, give-up word and *status set) and
 * the kernel still ends normally.  Process-wide; off by default. */
void mcv_testing_lm_head_skew_poll(int on);
int mcv_w4a16_lm_head_argmax_noalloc(const void* x_dev, int64_t K, int64_t N, int64_t V,
                                     const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                                     int zero_bias, void* logits_dev, int64_t* token_dev,
                                     uint32_t* status, mcv_stream_t stream);

/* The greedy lm_head with the last step of the argmax left to the reader of
 * the token, for callers that copy the token to the host anyway (the
 * reference's lm_head_greedy returns it to the host, language_model.cpp:
 * 464-481).  The kernel is the one above, but each workgroup ends with one
 * fire-and-forget atomicMax of a key tagged with `tag` into one of
 * MCV_LM_SLOTS slots (MCV_LM_SLOT_STRIDE u64 words apart) of slots_dev
 * (mcv_lm_head_slots_bytes() bytes, 128-byte aligned), so no workgroup waits
 * on a device round trip.  Copy the slots to the host and call
 * mcv_lm_head_slots_token(slots, tag) for the token (same value and tie rule
 * as mcv_w4a16_lm_head_argmax).  Tags: zero-fill the slots once, then give
 * every call a tag in [1, MCV_LM_SLOT_TAG_MAX] larger than any tag used since
 * the last zero-fill (zero-fill again before wrapping).  V < 2^24.  Calls
 * sharing one slots buffer must not overlap. */
#define MCV_LM_SLOTS 64
#define MCV_LM_SLOT_STRIDE 16
#define MCV_LM_SLOT_TAG_MAX 0xffffffu
int64_t mcv_lm_head_slots_bytes(void);
int mcv_w4a16_lm_head_argmax_slots(const void* x_dev, int64_t K, int64_t N, int64_t V,
                                   const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                                   int zero_bias, void* logits_dev, void* slots_dev, uint32_t tag,
                                   mcv_stream_t stream);
/* Host: the token from a host copy of the slots; never fails on valid slots. */
int64_t mcv_lm_head_slots_token(const uint64_t* slots_host, uint32_t tag);

/* The same greedy lm_head in two launches, for callers that fold the final
 * key reduction into their own next kernel: the GEMV writes logits (may be
 * NULL) and one 64-bit argmax key per 64-column slab to keys_dev (8-byte
 * aligned, 8 * ceil(V / 64) bytes, no initialisation needed);
 * mcv_argmax_reduce_keys folds n_keys keys into the int64 token.  A key orders
 * by fp16 value (subnormals as zero, NaN and -inf never winning), then by the
 * smaller column index. */
int mcv_w4a16_gemv_argmax_partials(const void* x_dev, int64_t K, int64_t N, int64_t V,
                                   const void* qw_dev, const void* scales_dev, const void* zeros_dev,
                                   int zero_bias, void* logits_dev, void* keys_dev, mcv_stream_t stream);
int mcv_argmax_reduce_keys(const void* keys_dev, int64_t n_keys, int64_t* token_dev, mcv_stream_t stream);

/* ------------------------------------------------------- W8A8 on device -- */
/* Per-row symmetric int8 activation quantisation: scale = max|x| / 127
 * (floor 1e-8), q = trunc(clamp(x * (1/scale), -128, 127) +- 0.5).
 * Replaces w8a8_quantize (src/csrc/lib/ops.cpp:1135-1171, kernel
 * op_kernel/w8a8_quantize_custom.cpp:18-47), which accepts M = 1 only.
 * x_scale_f32_dev [M] receives the fp32 scale and x_scale_f16_dev [M] its fp16
 * RNE encoding, the reference's stored form; either (not both) may be NULL. */
int mcv_w8a8_quantize_act(const void* x_dev, int64_t M, int64_t K, int8_t* xq_dev,
                          float* x_scale_f32_dev, void* x_scale_f16_dev, mcv_stream_t stream);

/* RMSNorm then per-row activation quantisation in one launch: the decode
 * sequence rms_norm -> w8a8_quantize that precedes every W8A8 projection
 * group (src/csrc/lib/decoder_layer.cpp:955-966, 1022-1032).  normed_dev
 * [M][H] fp16 receives the normed row (as mcv_rms_norm; may be NULL when no
 * fp16 consumer remains); xq_dev and the scales as mcv_w8a8_quantize_act of
 * that row.  Bit-identical to mcv_rms_norm followed by mcv_w8a8_quantize_act. */
int mcv_rms_norm_w8a8_quantize(const void* x_dev, const void* gamma_dev, int64_t M, int64_t H, double eps,
                               void* normed_dev, int8_t* xq_dev, float* x_scale_f32_dev,
                               void* x_scale_f16_dev, mcv_stream_t stream);

/* acc[M][N] int32 = xq[M][K] . W exactly.  W is int8 in layout w_layout.
 * Replaces matmul_w8a8_i32 (src/csrc/lib/ops.cpp:1097-1133, kernel
 * op_kernel/matmul_w8a8_i32_custom.cpp:15-48), which accepts M = 1 only.
 * MCV_W8_TILED runs the operand-line GEMV (M <= 4; M <= 2 when K > 2048) or
 * GEMM (larger M); the
 * KN / NK layouts a slower kernel that transposes through LDS. */
int mcv_w8a8_gemm_i32(const int8_t* xq_dev, int64_t M, int64_t K, int64_t N,
                      const int8_t* w_dev, int w_layout, int32_t* acc_dev, mcv_stream_t stream);

/* Dequant epilogue: out = fp16 RNE(((float)acc * w_scale[n]) * x_scale[m]).
 * Scales are fp32 or fp16 (mcv_dtype).  Replaces w8a8_dequant
 * (src/csrc/lib/ops.cpp:1173-1210, op_kernel/w8a8_dequant_custom.cpp:33-69). */
int mcv_w8a8_dequant(const int32_t* acc_dev, const void* x_scale_dev, int x_scale_dtype,
                     const void* w_scale_dev, int w_scale_dtype, int64_t M, int64_t N,
                     void* out_dev, mcv_stream_t stream);

/* Fused int8 GEMM + dequant epilogue: the int32 accumulator never leaves the
 * chip.  Bit-identical to mcv_w8a8_gemm_i32 followed by mcv_w8a8_dequant.
 * Replaces the matmul_w8a8_i32 + w8a8_dequant pair of
 * matmul_decode_w8a8_prequant (src/csrc/lib/decoder_layer.cpp:216-224). */
int mcv_w8a8_gemm_f16(const int8_t* xq_dev, const void* x_scale_dev, int x_scale_dtype,
                      int64_t M, int64_t K, int64_t N, const int8_t* w_dev, int w_layout,
                      const void* w_scale_dev, int w_scale_dtype, void* out_dev,
                      mcv_stream_t stream);

/* The int8 MFMA GEMM behind mcv_w8a8_gemm_i32 / _f16 for M > 4 on
 * MCV_W8_TILED weights, with an explicit tile configuration instead of the
 * dispatch's (no counterpart in the reference; exposed so every built
 * configuration can be tested and timed): bm x bn tiles (128x128, 64x128,
 * 128x64, 64x64), `stages` 128-k stages in flight (3 or 4),
 * `weights_in_registers` 1 to have each of the four waves load its own weight
 * columns into registers (128x128 and 64x128 only; LDS then stages x alone).
 * f16_out 1: fp16 out through the fused epilogue (scales as mcv_w8a8_gemm_f16),
 * 0: int32 out (scales unused).  An unbuilt configuration fails with
 * MCV_ERR_INVALID_ARG. */
int mcv_w8a8_gemm_lds(const int8_t* xq_dev, const void* x_scale_dev, int x_scale_dtype,
                      int64_t M, int64_t K, int64_t N, const int8_t* w_dev, const void* w_scale_dev,
                      int w_scale_dtype, void* out_dev, int f16_out, int bm, int bn, int stages,
                      int weights_in_registers, mcv_stream_t stream);

/* The whole W8A8 decode MLP block, M = 1, in one launch, from the normed fp16
 * row x [1][H]: quantise x, gate and up int8 GEMVs with the fused epilogue,
 * silu * mul, quantise the act row, the down int8 GEMV with its epilogue ->
 * out fp16 [1][H] (the decoder layers' W8A8 MLP sequence,
 * src/csrc/lib/decoder_layer.cpp:1022-1046).  Weights are MCV_W8_TILED
 * (gate/up H x I, down I x H); H <= 8192, I <= 16384, H and I multiples of 128.
 * scale_dtype MCV_F16: the weight scales are the reference's fp16 w_scale
 * (truncating encode) and every epilogue uses the activation scale rounded to
 * fp16, as the reference's w8a8_quantize stores it -- bit-identical to
 * mcv_w8a8_quantize_act, mcv_w8a8_gate_up_silu, mcv_w8a8_quantize_act,
 * mcv_w8a8_gemm_f16 with fp16 scales, i.e. the reference's precision.
 * MCV_F32: fp32 weight and activation scales throughout (the same sequence
 * with fp32 scales).  Values pass between workgroups through `workspace_dev`
 * (mcv_w8a8_mlp_workspace_bytes(H, I) bytes, 256-byte aligned, zero-filled
 * once; one shape per workspace; calls sharing it must not overlap); waits
 * give up as in mcv_w4a16_mlp, flagging the workspace's u32 at byte 0 and
 * `*status` (may be NULL).  MCV_ERR_SHAPE when the launch would not fit on
 * the device at once. */
int64_t mcv_w8a8_mlp_workspace_bytes(int64_t H, int64_t I);
int mcv_w8a8_mlp(const void* x_dev, int64_t H, int64_t I, const int8_t* w_gate_dev, const void* ws_gate_dev,
                 const int8_t* w_up_dev, const void* ws_up_dev, const int8_t* w_down_dev, const void* ws_down_dev,
                 int scale_dtype, void* out_dev, void* workspace_dev, uint32_t* status, mcv_stream_t stream);

/* Decode MLP front half over W8A8 weights: act[M][N] fp16 = silu(gate) * up,
 * gate and up each the fused epilogue of mcv_w8a8_gemm_f16 over the same
 * quantised x (one activation quantisation shared by both, as
 * decoder_layer.cpp:1029-1046 does).  Both weights MCV_W8_TILED [K][N], their
 * scales in ws_dtype; M in [1, 4].  One launch, bit-identical to two
 * mcv_w8a8_gemm_f16 calls and mcv_silu_mul. */
int mcv_w8a8_gate_up_silu(const int8_t* xq_dev, const void* x_scale_dev, int x_scale_dtype, int64_t M,
                          int64_t K, int64_t N, const int8_t* w_gate_dev, const void* w_scale_gate_dev,
                          const int8_t* w_up_dev, const void* w_scale_up_dev, int w_scale_dtype, void* act_dev,
                          mcv_stream_t stream);

/* W8A8 lm_head, step one of two (M = 1): logits[v] = the fused epilogue of
 * mcv_w8a8_gemm_f16 over the MCV_W8_TILED weight [K][N] for v < V (bit-
 * identical to it; logits_dev may be NULL), and one first-maximum argmax key
 * per 64-column slab into keys_dev (ceil(V / 64) u64, 8-byte aligned), as
 * mcv_w4a16_gemv_argmax_partials writes them; mcv_argmax_reduce_keys(keys_dev,
 * ceil(V / 64), token_dev) finishes.  Replaces the W8A8 branch of
 * lm_head_greedy (src/csrc/lib/language_model.cpp:434-480: 16 chunk
 * matmul_w8a8 + w8a8_dequant launches, their D2H copies and the host scan). */
int mcv_w8a8_gemv_argmax_partials(const int8_t* xq_dev, const void* x_scale_dev, int x_scale_dtype, int64_t K,
                                  int64_t N, int64_t V, const int8_t* w_dev, const void* w_scale_dev,
                                  int w_scale_dtype, void* logits_dev, void* keys_dev, mcv_stream_t stream);

/* The whole W8A8 lm_head step in one launch (M = 1): the activation row x_dev
 * (fp16 [K], K a multiple of 16 up to 2048) quantised as mcv_w8a8_quantize_act
 * does it, the GEMV
 * over the MCV_W8_TILED weight [K][N] with the fused epilogue for v < V
 * (logits_dev, may be NULL) and the first-maximum argmax as an int64 token on
 * the device -- bit-identical to mcv_w8a8_quantize_act +
 * mcv_w8a8_gemv_argmax_partials + mcv_argmax_reduce_keys with the same scale
 * dtypes.  x_scale_dtype MCV_F16: the epilogue multiplies by the fp16 x_scale
 * the reference stores (language_model.cpp:439-441); w_scale in
 * w_scale_dtype.  The workspace is mcv_w4a16_lm_head_argmax's
 * (mcv_lm_head_workspace_bytes(V), 128-byte aligned, zero-filled once; the
 * same generation word, key words and give-up word, so the two heads may
 * share one, one call at a time).  MCV_ERR_SHAPE above K = 2048 (the three
 * launches then serve).  Replaces the W8A8 branch of lm_head_greedy
 * (src/csrc/lib/language_model.cpp:434-480). */
/* The grid mcv_w8a8_lm_head_argmax launches for V: slabs of 64 columns per
 * workgroup (4 from V = 130817 up, 2 from V = 65409, else 1); 0 for an
 * unsupported V. */
int64_t mcv_w8a8_lm_head_slabs_per_workgroup(int64_t V);

int mcv_w8a8_lm_head_argmax(const void* x_dev, int64_t K, int64_t N, int64_t V, const int8_t* w_dev,
                            const void* w_scale_dev, int w_scale_dtype, int x_scale_dtype, void* logits_dev,
                            int64_t* token_dev, void* workspace_dev, uint32_t* status, mcv_stream_t stream);

/* Bytes of a K x N weight in MCV_W8_TILED (0 on bad shape). */
int64_t mcv_w8a8_tiled_bytes(int64_t K, int64_t N);

/* Re-lays an int8 [K][N] weight (the reference's w_int8 layout) into
 * MCV_W8_TILED on the host; tiled_host holds mcv_w8a8_tiled_bytes(K, N). */
int mcv_w8a8_pack_tiled_host(const int8_t* q_kn_host, int64_t K, int64_t N, int8_t* tiled_host);

/* Host-side per-output-channel weight quantiser: replaces
 * quantize_dense_weight_w8a8 (src/csrc/lib/quantized_weight.cpp:231-268) minus
 * its device round trip.  w_kn_host fp16 [K][N]; q_host int8 in out_layout
 * (MCV_W8_TILED: mcv_w8a8_tiled_bytes(K, N) bytes);
 * scale_f32_host [N]; scale_f16_host [N] (truncating encode, :253), may be NULL. */
int mcv_w8a8_quantize_weight_host(const uint16_t* w_kn_host, int64_t K, int64_t N,
                                  int8_t* q_host, int out_layout, float* scale_f32_host,
                                  uint16_t* scale_f16_host);

/* Source element type of a checkpoint tensor. */
enum mcv_src_dtype {
    MCV_SRC_F16 = 0,
    MCV_SRC_BF16 = 1  /* converted as the reference loads bf16 (src/csrc/lib/weights.cpp:25-33) */
};

/* The same per-output-channel quantiser fed straight from a checkpoint's
 * [N][K] (out, in) linear weight, fp16 or bf16, in one host pass: replaces
 * the reference's bf16 load, host transpose and quantisation
 * (load_matmul_weight_transposed, src/csrc/lib/language_model.cpp:84-105,
 * then quantize_dense_weight_w8a8, quantized_weight.cpp:231-268), bit-identical
 * to them.  Outputs as mcv_w8a8_quantize_weight_host. */
int mcv_w8a8_quantize_weight_nk_host(const uint16_t* w_nk_host, int src_dtype, int64_t K, int64_t N,
                                     int8_t* q_host, int out_layout, float* scale_f32_host,
                                     uint16_t* scale_f16_host);
/* The same from [N_src][K] rows into N >= N_src output channels, channels
 * from N_src on zero (scale 1e-8, q = 0): the tied embedding [vocab, hidden]
 * quantised as the reference quantises its zero-padded lm_head chunks
 * (src/csrc/lib/language_model.cpp:238-270). */
int mcv_w8a8_quantize_weight_nk_pad_host(const uint16_t* w_nk_host, int src_dtype, int64_t K, int64_t N_src,
                                         int64_t N, int8_t* q_host, int out_layout, float* scale_f32_host,
                                         uint16_t* scale_f16_host);

/* Re-lays a pre-quantised int8 [N][K] checkpoint tensor (safetensors I8, no
 * counterpart in the reference, whose loader has no I8 dtype,
 * src/csrc/lib/weights.cpp:15-23) into MCV_W8_TILED on the host. */
int mcv_w8a8_pack_tiled_nk_host(const int8_t* q_nk_host, int64_t K, int64_t N, int8_t* tiled_host);

/* The kernel the W8A8 GEMM entry points launch for M x K x N with a weight in
 * `w_layout` (fp16 output through the fused epilogue when out_f16, else
 * int32), as text with its template arguments as a kernel trace names them
 * (the epilogue argument as launched with fp32 scales), for labels in
 * reports; valid until the next call on this thread.  No reference
 * counterpart. */
const char* mcv_w8a8_gemm_kernel_name(int64_t M, int64_t K, int64_t N, int w_layout, int out_f16);

/* ------------------------------------------------------------ elementwise -- */
/* out = fp16 RNE(silu(g) * u) in fp32, n elements.  Replaces silu_mul
 * (src/csrc/lib/ops.cpp:437-456, op_kernel/silu_mul_custom.cpp:38-89). */
int mcv_silu_mul(const void* gate_dev, const void* up_dev, void* out_dev, int64_t n,
                 mcv_stream_t stream);

/* Per-row argmax of fp16 [M][N] into int64 [M], first maximum wins, fp16
 * subnormals compare as zero, NaN never wins.  Replaces argmax_last_dim
 * (src/csrc/lib/ops.cpp:324-355) with the tie rule of lm_head_greedy
 * (src/csrc/lib/language_model.cpp:473-479). */
int mcv_argmax_f16(const void* x_dev, int64_t M, int64_t N, int64_t* idx_dev,
                   mcv_stream_t stream);

/* Row-wise RMSNorm of fp16 [M][H]: y = fp16 RNE((x * rstd) * gamma) with
 * rstd = 1 / sqrt(mean(x^2) + eps) in fp32.  The final norm that
 * lm_head_greedy applies before the vocabulary projection
 * (src/csrc/lib/language_model.cpp:424, an aclnn builtin in the reference). */
int mcv_rms_norm(const void* x_dev, const void* gamma_dev, int64_t M, int64_t H, double eps, void* out_dev,
                 mcv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MCV_QUANT_H */
