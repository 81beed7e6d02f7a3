/*
 * vcx.h -- C ABI of the MI355X (gfx950) sageattn_vc implementation.
 *
 * The library libvcx.so (built from cake-opt-vc_attention_amd/csrc) exports
 * exactly the functions declared here. Every entry point:
 *   - takes raw device pointers plus explicit shapes and element strides;
 *   - never allocates: the caller owns every output and workspace buffer;
 *   - enqueues all work on the given HIP stream (hipStream_t passed as void*;
 *     NULL means the null stream) and never synchronizes;
 *   - launches on the calling thread's current HIP device: the stream and every
 *     pointer must belong to that device;
 *   - returns VCX_OK (0) or a nonzero error code, with a message available
 *     from vcx_last_error() on the calling thread; no C++ exception crosses
 *     this boundary;
 *   - validates shapes, strides, alignment and sizes before any launch.
 *
 * Tensor conventions (B batch, H heads, N tokens, D head dim in {64,128}):
 *   q, k, v        fp16/bf16, element strides (sb, sh, sn), unit stride over D;
 *                  HND and NHD layouts are both expressed by these strides.
 *   q8 / k8        int8 [B,H,N,D] contiguous (logical token order; k8 is in
 *                  permuted order when a permutation is given).
 *   qs             fp32 [B,H,ceil(Nq/64)*32], index (row/16)*8 + row%8.
 *   ks             fp32 [B,H,ceil(Nk/128)*4], index tile*4 + (key%8)/2.
 *   v8             E4M3 bytes [B,H,D,ceil(Nk/128)*128] in STORAGE order: inside
 *                  every 128-token tile, byte position p holds token
 *                  vcx_value_token(p) (see below); padding tokens are 0x00.
 *   vs             fp32 [B,H,D] (per-channel) or [B,H,tiles,D] (per-block).
 *   means          binary16 [B,H,tiles,D] (V smoothing only).
 */
#ifndef VCX_H
#define VCX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VCX_ABI_VERSION 3
#define VCX_CLOCK_PROBE_BLOCKS 8
#define VCX_NOALLOC_SCRATCH_BYTES (32u << 20) /* scratch of vcx_prepare_qk_int8_noalloc, per GPU */

enum vcx_status {
  VCX_OK = 0,
  VCX_EINVAL = 1,       /* invalid argument, shape, stride, alignment or size */
  VCX_EUNSUPPORTED = 2, /* valid request this build does not implement */
  VCX_EHIP = 3          /* a HIP runtime call failed */
};

enum vcx_dtype { VCX_FLOAT16 = 0, VCX_BFLOAT16 = 1, VCX_FLOAT32 = 2 /* vcx_preprocess_qk only */ };

enum vcx_group_mode {
  VCX_GROUP_AUTO = 0,   /* fused schedule for <= 8 effective clusters, general above (group_values) */
  VCX_GROUP_GENERAL = 1 /* general schedule for every count (group_values_legacy) */
};

enum vcx_workspace_op {
  VCX_WS_PREPARE_QK = 1, /* vcx_prepare_qk_int8 */
  VCX_WS_PREPARE_V = 2,  /* vcx_prepare_v_fp8 (smoothing off or on) */
  VCX_WS_GROUP = 3,      /* vcx_group_values */
  VCX_WS_PREPROCESS_QK = 4 /* vcx_preprocess_qk (k_smooth = 1); any D in 1..128 */
};

/* Library ABI version (VCX_ABI_VERSION). Replaces the reference's build-stamp
 * attributes sage_vc_api_version / sage_vc_kernel_version checked at
 * third_party/sageattention_local/sageattention_local/vc.py:49-55. */
int vcx_abi_version(void);

/* Message of the last failing call on this thread ("" if none). Replaces the
 * TORCH_CHECK messages of third_party/sageattention_local/csrc/vc/vc_sm90.cu:1030-1064. */
const char* vcx_last_error(void);

/* Storage position -> token offset inside a 128-token V tile (p in 0..127).
 * The reference stores Sage's 16-token permutation instead
 * (third_party/sageattention_local/sageattention_local/vc_reference.py:14-17,
 * csrc/fused/fused.cu:287-291); this order feeds the gfx950 FP8 MFMA B layout. */
int vcx_value_token(int p);

/* Bytes of caller-provided workspace needed by one call of the given op.
 * clusters matters for VCX_WS_GROUP only (either mode); smooth for VCX_WS_PREPARE_V. */
int vcx_workspace_bytes(int op, int64_t B, int64_t H, int64_t N, int64_t D, int smooth,
                        int clusters, size_t* bytes);

/* V grouping: count = min(clusters, N) in 1..256 clusters per head, `iterations` Lloyd
 * passes (fp64 distances, ties to the lowest id, empty clusters keep their center, center
 * sums in fp64 tile order), then a stable counting sort by label. mode VCX_GROUP_AUTO runs
 * the fused schedule for count <= 8 and the general one above; VCX_GROUP_GENERAL runs the
 * general one for every count (same results where both apply).
 * centers_in (nullable, fp32 [B,H,count,D]): initial centers (the warm start of a cached
 * layout); NULL starts from V[trunc(fp32 linspace(0, N-1, count))].
 * Outputs: perm int64 [B,H,N]; labels int32 [B,H,N] (nullable); centers fp32
 * [B,H,count,D] used by the final assignment (nullable); centers_next fp32 [B,H,count,D]
 * (nullable): the Lloyd update of the final labels, to pass as centers_in next time.
 * Replaces _vc_sm90.group_values / group_values_debug / group_values_legacy(_debug)
 * (third_party/sageattention_local/csrc/vc/pybind.cpp:6-44, clustering.cu:140-167) and the
 * warm-started grouping of src/vc_attention/core.py:153-171 (cuda_backend.py:24-25). */
int vcx_group_values(const void* v, int dtype, int64_t B, int64_t H, int64_t N, int64_t D,
                     int64_t v_sb, int64_t v_sh, int64_t v_sn, int clusters, int iterations, int mode,
                     const float* centers_in, int64_t* perm, int32_t* labels, float* centers,
                     float* centers_next, void* workspace, size_t workspace_bytes, void* stream);

/* Q/K INT8 with Sage per-thread scales, after K channel-mean centring.
 * perm (nullable, int64 [B,H,Nk]) gathers K tokens first. km_out (nullable)
 * receives the channel mean [B,H,D] in the input dtype.
 * Replaces `km = k.mean(2); per_thread_int8(q, k, km, BLKQ=64, WARPQ=16,
 * BLKK=128, WARPK=128)` (third_party/sageattention_local/sageattention_local/vc.py:155-159,
 * triton/quant_per_thread.py:154-204). */
int vcx_prepare_qk_int8(const void* q, const void* k, int dtype, int64_t B, int64_t H,
                        int64_t Nq, int64_t Nk, int64_t D, int64_t q_sb, int64_t q_sh,
                        int64_t q_sn, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                        const int64_t* perm, int8_t* q8, float* qs, int8_t* k8, float* ks,
                        void* km_out, void* workspace, size_t workspace_bytes, void* stream);

/* vcx_prepare_qk_int8 without a workspace argument and without any allocation: the K tile
 * sums and mean live in a file-scope device array of VCX_NOALLOC_SCRATCH_BYTES (32 MiB) per
 * GPU, held until the process ends. Same arguments (minus the workspace),
 * outputs and results as vcx_prepare_qk_int8; shapes whose ws_prepare_qk workspace
 * (8*B*H*ceil(Nk/128)*D + 4*B*H*D bytes, 256-byte aligned slices) exceeds the scratch are
 * rejected with VCX_EINVAL. All calls on one GPU share the scratch: calls that overlap on one
 * GPU (concurrent streams or threads) race. The array's device address is resolved once per
 * device (hipGetSymbolAddress on the first call there) and kept: a hipDeviceReset or an
 * unload of the library's code object in the same process invalidates it, so such a
 * process must not call this entry point afterwards. No counterpart in the reference; for
 * callers that cannot allocate (code under HIP graph capture, allocation-free serving loops). */
int vcx_prepare_qk_int8_noalloc(const void* q, const void* k, int dtype, int64_t B, int64_t H,
                                int64_t Nq, int64_t Nk, int64_t D, int64_t q_sb, int64_t q_sh,
                                int64_t q_sn, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                                const int64_t* perm, int8_t* q8, float* qs, int8_t* k8, float* ks,
                                void* km_out, void* stream);

/* vcx_prepare_qk_int8 with Q and the centred K rotated by the normalized Sylvester-
 * Hadamard transform before the INT8 quantizer: q' = H(q), k' = H(RN_in(k - km)), in
 * binary32 with butterflies of stride 1, 2, 4, ... ((a + b, a - b), each RN) and a final
 * multiply by RN_f32(1/sqrt(D)); not rounded back to the input dtype. Same arguments,
 * outputs and workspace as vcx_prepare_qk_int8. No counterpart inside the reference's
 * sageattn_vc, whose H200_INT8.md:99-104 names the rotation as its remaining gap; the
 * transform is the reference's (src/vc_attention/core.py:79-107, csrc/kernels.cu:104-123). */
int vcx_prepare_qk_int8_rotated(const void* q, const void* k, int dtype, int64_t B, int64_t H,
                                int64_t Nq, int64_t Nk, int64_t D, int64_t q_sb, int64_t q_sh,
                                int64_t q_sn, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                                const int64_t* perm, int8_t* q8, float* qs, int8_t* k8, float* ks,
                                void* km_out, void* workspace, size_t workspace_bytes, void* stream);

/* Post-RoPE Q/K preprocessing in binary32: inputs (fp16, bf16 or fp32; D in 1..128; strided)
 * are widened; k_smooth subtracts K's binary32 channel mean RN_f32(S/Nk) (S the binary64 sum
 * per 128-key tile in key order, then over tiles in order); hadamard rotates Q and K rows as
 * above with W = the power of two >= D (zero padded). Outputs q_out [B,H,Nq,W'] and
 * k_out [B,H,Nk,W'] binary32 contiguous, W' = hadamard ? W : D. Workspace
 * VCX_WS_PREPROCESS_QK when k_smooth (else nullable).
 * Replaces the reference's preprocess_qk (csrc/bindings.cpp:87-116, kernels.cu:104-123,396-405). */
int vcx_preprocess_qk(const void* q, const void* k, int dtype, int64_t B, int64_t H, int64_t Nq,
                      int64_t Nk, int64_t D, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb,
                      int64_t k_sh, int64_t k_sn, int k_smooth, int hadamard, float* q_out,
                      float* k_out, void* workspace, size_t workspace_bytes, void* stream);

/* Q/K block-scaled E4M3 (the experimental vc27 QK format). K is centred by its
 * binary32 channel mean km = RN_f32(S/Nk) (S the fp64 sum in this library's fixed
 * tile-tree order); Q in 64-row blocks, centred K in 128-row blocks, each block with
 * one scale s = max(RN(amax/448), 1e-12) and codes E4M3_satfinite(RN(x/s)).
 * Outputs: q8 [B,H,Nq,D], qs fp32 [B,H,ceil(Nq/64)], k8 [B,H,Nk,D], ks fp32
 * [B,H,ceil(Nk/128)], km_out (nullable) fp32 [B,H,D]. Workspace: VCX_WS_PREPARE_QK.
 * Replaces _vc_sm90.prepare_qk_fp8 (third_party/sageattention_local/csrc/vc/pybind.cpp:56,
 * qk_fp8.cu:10-109). */
int vcx_prepare_qk_fp8(const void* q, const void* k, int dtype, int64_t B, int64_t H,
                       int64_t Nq, int64_t Nk, int64_t D, int64_t q_sb, int64_t q_sh,
                       int64_t q_sn, int64_t k_sb, int64_t k_sh, int64_t k_sn, uint8_t* q8,
                       float* qs, uint8_t* k8, float* ks, float* km_out, void* workspace,
                       size_t workspace_bytes, void* stream);

/* V to E4M3. smooth = 0: per-channel amax scale (vs [B,H,D], means unused).
 * smooth = 1: 128-token block-mean residuals with per-channel (channel_scale=1,
 * vs [B,H,D]) or per-block (channel_scale=0, vs [B,H,tiles,D]) scales and
 * binary16 scaled means [B,H,tiles,D]. perm (nullable) gathers tokens first.
 * Replaces per_channel_fp8 (third_party/sageattention_local/sageattention_local/quant.py:224-293,
 * with the zero padding of vc.py:163-166) and _vc_sm90.prepare_values
 * (third_party/sageattention_local/csrc/vc/preprocess.cu:138-168). */
int vcx_prepare_v_fp8(const void* v, int dtype, int64_t B, int64_t H, int64_t N, int64_t D,
                      int64_t v_sb, int64_t v_sh, int64_t v_sn, const int64_t* perm, int smooth,
                      int channel_scale, uint8_t* v8, float* vs, uint16_t* means,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Fused attention forward: INT8 QK^T on MFMA, ExpCast E4M3 probabilities,
 * FP8 PV on MFMA, online max/sum, block-mean restore, epilogue.
 * expcast = 1: unfused ExpCast bytes (the reference's oracle and vc4..vc11 modes).
 * expcast = 2: the folded ExpCast encode of the reference's default modes
 * (vc12..vc15, "optimized"; vc_math.cuh:16-111), only with block_values = 0, with the
 * reference's per-16-row-group fallback to the unfused bytes when some |m'| > 128.
 * expcast = 0: the Sage FP8 control path, P = E4M3 of the correctly rounded binary32
 * exp2 (v_exp_f32, rechecked in binary64 where an E4M3 rounding midpoint lies within two
 * ulps; the bytes are exact) with the 8.807 offset, and the unrounded v_exp_f32 values
 * summed as the row mass. block_values = 1 consumes means/vs as written by
 * vcx_prepare_v_fp8(smooth=1, channel_scale): channel_scale = 1 applies vs
 * [B,H,D] in the epilogue, channel_scale = 0 scales every tile's contribution
 * by its vs [B,H,tiles,D]; block_values = 0 uses vs [B,H,D], ignores means and
 * requires channel_scale = 1. out: fp16/bf16 (out_dtype) with element strides.
 * p_dump (nullable): diagnostic copy of the E4M3 P bytes for query rows
 * [p_row_begin, p_row_end) of every head, uint8 [B,H,rows,ceil(Nk/128)*128]
 * in logical key order (padding keys 0); slower kernel variant.
 * Replaces _vc_sm90.forward (third_party/sageattention_local/csrc/vc/pybind.cpp:51-55,
 * vc_sm90.cu:1027-1123). */
int vcx_attention_fwd(const int8_t* q8, const int8_t* k8, const uint8_t* v8, const float* qs,
                      const float* ks, const float* vs, const uint16_t* means, int64_t B,
                      int64_t H, int64_t Nq, int64_t Nk, int64_t D, int expcast,
                      int block_values, int channel_scale, float sm_scale, int out_dtype,
                      void* out, int64_t o_sb, int64_t o_sh, int64_t o_sn, uint8_t* p_dump,
                      int64_t p_row_begin, int64_t p_row_end, void* stream);

/* Fused attention forward on block-scaled FP8 Q/K (vcx_prepare_qk_fp8): E4M3 QK^T on
 * v_mfma_f32_16x16x128_f8f6f4, logit scale RN(qs[row/64] * ks[tile]), then the same
 * probability paths, PV and epilogue as vcx_attention_fwd without block values. V is
 * the per-channel payload of vcx_prepare_v_fp8(smooth = 0) with vs [B,H,D].
 * expcast: 2 folded ExpCast encode (the reference's FP8 kernel), 1 unfused ExpCast,
 * 0 Sage FP8 control. q8 [B,H,Nq,D], k8 [B,H,Nk,D] E4M3 bytes; qs [B,H,ceil(Nq/64)];
 * ks [B,H,ceil(Nk/128)]. out, p_dump as for vcx_attention_fwd.
 * Replaces _vc_sm90.forward_fp8 (third_party/sageattention_local/csrc/vc/pybind.cpp:57,
 * fp8_dispatch.cuh:76-111). */
int vcx_attention_fwd_fp8(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8, const float* qs,
                          const float* ks, const float* vs, int64_t B, int64_t H, int64_t Nq,
                          int64_t Nk, int64_t D, int expcast, float sm_scale, int out_dtype,
                          void* out, int64_t o_sb, int64_t o_sh, int64_t o_sn, uint8_t* p_dump,
                          int64_t p_row_begin, int64_t p_row_end, void* stream);

/* ExpCast byte probe: y[i] = clamp(RNE(fmaf(x[i], 11.54156, 119.65)), 0, 120).
 * Replaces _vc_sm90.expcast_codes (third_party/sageattention_local/csrc/vc/preprocess.cu:170-179). */
int vcx_expcast_codes(const float* x, uint8_t* y, int64_t n, void* stream);

/* Control-path probability probe: y[i] = E4M3_RNE(RN_f32(exp2(x[i]))), the P byte of the
 * Sage FP8 control path (vcx_attention_fwd expcast = 0) computed by the fused kernel's own
 * device function (hardware exp2, rechecked in binary64 next to an E4M3 rounding midpoint);
 * form 1 forms the lower window neighbours by saturating subtraction (what the fused kernel
 * runs on every tile), form 0 by one 64-bit subtraction per pair (same bytes, more
 * rechecks for probabilities below two subnormal ulps).
 * Replaces the probability byte of third_party/sageattention_local/sageattention_local/
 * vc_reference.py:68-75 (torch.exp2 then float8_e4m3fn), for the parity tests. */
int vcx_fp8_exp2_codes(const float* x, uint8_t* y, int64_t n, int form, void* stream);

/* Diagnostic probe of the gfx950 conversions the kernels rely on:
 * u8[i] = v_cvt_pk_u8_f32(x[i]) and f8[i] = v_cvt_pk_fp8_f32(clamp(x[i], +-448)).
 * No counterpart in the reference (which probes only ExpCast); used by the
 * parity tests to pin the instructions' rounding against the CPU oracle. */
int vcx_convert_probe(const float* x, uint8_t* u8, uint8_t* f8, int64_t n, void* stream);

/* Compiled resources of the fused kernel for (D, block_values):
 * out[0] VGPRs, out[1] AGPRs (0 if not reported), out[2] static LDS bytes,
 * out[3] dynamic LDS bytes per block, out[4] threads per block,
 * out[5] scratch (spill) bytes per lane.
 * Replaces _vc_sm90.kernel_resources (third_party/sageattention_local/csrc/vc/vc_sm90.cu:786-822). */
int vcx_kernel_resources(int64_t D, int block_values, int64_t* out);

/* Compiled resources of the fused kernel that one launch mode runs: value_mode 0 (no
 * block values), 1 (block values, channel scales), 2 (block values, per-block scales);
 * expcast 0/1/2 as for vcx_attention_fwd (2 only with value_mode 0); out_dtype
 * VCX_FLOAT16 / VCX_BFLOAT16. out[0..5] as for vcx_kernel_resources, out[6] the
 * occupancy-predicted active blocks per CU (256 threads per block; a device call).
 * Replaces the per-mode entries of _vc_sm90.kernel_resources(output_type)
 * (third_party/sageattention_local/csrc/vc/vc_sm90.cu:786-822,1123-1160), which
 * sageattention_local.kernel_resources maps onto the reference's mode names. */
int vcx_kernel_resources_mode(int64_t D, int value_mode, int expcast, int out_dtype, int64_t* out);

/* The same six values for the FP8 block QK kernel (expcast = 1: folded ExpCast,
 * 0: control). Replaces _vc_sm90.fp8_kernel_resources
 * (third_party/sageattention_local/csrc/vc/fp8_dispatch.cuh:61-73). */
int vcx_kernel_resources_fp8(int64_t D, int expcast, int64_t* out);

/* Engine-clock probe: VCX_CLOCK_PROBE_BLOCKS one-wave blocks on `stream` (one per XCD
 * as the hardware deals blocks) each count s_memtime ticks (the engine clock) against
 * s_memrealtime ticks (constant rate, *wall_khz kHz) over window_us microseconds of real
 * time; block i stores out[2i] = engine ticks, out[2i+1] = real-time ticks (device
 * memory, 8-byte aligned); its clock = out[2i] / out[2i+1] * wall_khz kHz. Run beside
 * the fused kernel on a second stream it reads the clock under load.
 * No counterpart in the reference; for reporting MFMA roofline fractions at the
 * measured clock. */
int vcx_clock_probe(int64_t window_us, uint64_t* out, int* wall_khz, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VCX_H */
