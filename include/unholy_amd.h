/* C ABI of the gfx950 quantized-MoE library (libunholy_amd.so).
 *
 * Each kernel entry point wraps the C++ drop-in of the same name in namespace unholy::kernels
 * (the headers under include/unholy/kernels/), which keeps the reference's signatures, weight/scale layouts and pointer-table
 * semantics; the reference declaration each one replaces is cited per function (paths in the reference tree
 * ewtodd/unholy). Conventions: plain pointers and sizes; device pointers unless named h_*; bf16 = uint16_t;
 * e4m3 / e2m1 codes and e8m0 scale exponents = uint8_t; `stream` is a hipStream_t (NULL = the null stream).
 * Every function returns 0 on success and -1 on failure (invalid shape, HIP error); uh_last_error() then
 * holds the message of the calling thread's last failure. Launches are asynchronous: device faults surface at
 * the next synchronizing call.
 */
#ifndef UNHOLY_AMD_H
#define UNHOLY_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime (no reference counterpart: src/rt/hip.hpp's DeviceBuffer / UH_CHECK play this role there) ---- */
const char* uh_last_error(void);
int uh_version(void); /* the library version (a value, not a status) */
int uh_device_count(int* n);
int uh_set_device(int dev);
int uh_device_name(char* buf, int len);
int uh_malloc(void** p, size_t bytes);
int uh_free(void* p);
int uh_memcpy_h2d(void* dst, const void* h_src, size_t bytes);
int uh_memcpy_d2h(void* h_dst, const void* src, size_t bytes);
int uh_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int uh_memset(void* dst, int value, size_t bytes, void* stream);
int uh_synchronize(void);
int uh_stream_create(void** stream);
int uh_stream_destroy(void* stream);
int uh_stream_synchronize(void* stream);
int uh_event_create(void** ev);
int uh_event_destroy(void* ev);
int uh_event_record(void* ev, void* stream);
int uh_event_synchronize(void* ev);
int uh_event_elapsed_ms(float* ms, void* start, void* stop);
/* Synthetic data on the device: n bytes of a splitmix64 stream (seed), each byte mapped to lo + (v % (hi-lo+1)). */
/* HIP graphs of a created stream's work (launch-bound sequences of short kernels): capture begin / end (the end
 * instantiates the graph and returns its executable), launch, destroy. */
int uh_graph_capture_begin(void* stream);
int uh_graph_capture_end(void* stream, void** exec);
int uh_graph_launch(void* exec, void* stream);
int uh_graph_destroy(void* exec);
int uh_fill_random_bytes(void* dst, size_t n, uint64_t seed, uint32_t lo, uint32_t hi, void* stream);

/* ---- MXFP4 layout and activation transforms (src/kernels/mx_moe.hpp) ---- */
/* mx_moe.hpp:27 */
int uh_mx_repack(uint8_t* w, uint8_t* s, int N, int K, uint8_t* tmp, void* stream);
/* mx_moe.hpp:29 */
int uh_mx_repack_to(const uint8_t* w, const uint8_t* s, uint8_t* tw, uint8_t* ts, int N, int K, void* stream);
/* mx_moe.hpp:33-34 (x_rows may be NULL) */
int uh_mx_xform_in(const uint16_t* x, int ldx, const int32_t* row_expert, const uint8_t* const* s_tab, uint16_t* xa,
                   int P, int K, void* stream, const int32_t* x_rows);
/* mx_moe.hpp:36-40: xa rows [plan[1], plan[0]) of resident experts rebuilt from compact fp8 token rows q [U, K] /
 * s [U, K/128] of token p2u[r]; the _fp8 form (no reference counterpart) copies the codes / exponents to pair rows of
 * qo [P, K] / qso [P, K/128] instead. */
int uh_mx_xform_in_q(const uint8_t* q, const uint8_t* s, const int32_t* p2u, const int32_t* plan,
                     const int32_t* row_expert, const uint8_t* const* s_tab, uint16_t* xa, int P, int K, void* stream);
int uh_mx_xform_in_q_fp8(const uint8_t* q, const uint8_t* s, const int32_t* p2u, const int32_t* plan,
                         const int32_t* row_expert, const uint8_t* const* s_tab, uint8_t* qo, uint8_t* qso, int P,
                         int K, void* stream);
/* No reference counterpart: mx_xform_in emitting e4m3 codes [P, K] + e8m0 scales [P, K/128] (the MFMA operand). */
int uh_mx_xform_in_fp8(const uint16_t* x, int ldx, const int32_t* row_expert, const uint8_t* const* s_tab,
                       uint8_t* q, uint8_t* qs, int P, int K, void* stream, const int32_t* x_rows);
/* mx_moe.hpp:41-42 */
int uh_mx_swiglu(const uint16_t* g, const uint16_t* u, const float* w, const int32_t* row_expert,
                 const uint8_t* const* s_tab, uint16_t* hh, int P, int I, float limit, void* stream);
/* No reference counterpart: exhaustive check of the hardware e4m3 encode (v_cvt_pk_fp8_f32) against the
 * software round-to-nearest-even encode on every fp32 value in [-448, 448]; *bad = mismatching codes. */
int uh_check_fp8_encode(unsigned long long* bad, unsigned long long* total);
/* No reference counterpart: exhaustive check of the hardware bf16 rounding (v_cvt_pk_bf16_f32) against the software
 * round-to-nearest-even over all 2^32 fp32 bit patterns; *bad = mismatches at non-NaN inputs plus NaN inputs whose
 * result is not a NaN, *nan_bad = NaN inputs whose NaN payload differs. */
int uh_check_bf16_encode(unsigned long long* bad, unsigned long long* nan_bad);
/* No reference counterpart: y[i] = e^x[i] as the SwiGLU epilogues and the softmax / sigmoid routers compute it (IEEE
 * operations only, the same bits as the CPU oracle's), for checks. */
int uh_exp_f32_array(const float* x, float* y, size_t n, void* stream);
/* mx_moe.hpp:61: exhaustive MFMA block-scaled decode check; *bad = mismatches among normal results. */
int uh_mx_check_dequant(unsigned long long* bad, unsigned long long* total);

/* ---- grouped expert GEMV / GEMM (src/kernels/mx_moe.hpp). tiles: int32 triples {expert, row0, rows}, ntiles of
 * them (the grid's tile count, as the reference launches it); with ntiles_dev the tiles at or past the device count
 * are read but not used, so the buffer holds ntiles entries either way.
 * glu_*: the MxGlu epilogue (glu_hh / glu_hq NULL: none); glu_hq + glu_hs: hh as e4m3 codes + e8m0 scales. ---- */
/* mx_moe.hpp:100-104 */
int uh_mx_grouped_gemv(const uint16_t* xa, int K, const int32_t* tiles, int ntiles, const uint8_t* const* w_tab,
                       const uint8_t* const* s_tab, uint16_t* out, int ldo, int N, void* stream,
                       const int* ntiles_dev, const uint8_t* const* w_tab2, const uint8_t* const* s_tab2,
                       uint16_t* out2, int max_rows, const float* glu_w, const int32_t* glu_row_expert,
                       const uint8_t* const* glu_s_tab, uint16_t* glu_hh, float glu_limit, uint32_t* glu_counters);
/* mx_moe.hpp:90-96, 100-104: uh_mx_grouped_gemv with the MxSums epilogue: sums_dst [U, N] = bf16 sums of each
 * compact token's remote pair rows (sums_u2p [U, sums_K], U = sums_plan[4]) of out (N % 128). */
int uh_mx_grouped_gemv_sums(const uint16_t* xa, int K, const int32_t* tiles, int ntiles, const uint8_t* const* w_tab,
                            const uint8_t* const* s_tab, uint16_t* out, int ldo, int N, void* stream,
                            const int* ntiles_dev, int max_rows, const int32_t* sums_u2p, const int32_t* sums_plan,
                            int sums_K, uint16_t* sums_dst, uint32_t* sums_counters);
/* mx_moe.hpp:49-52 */
int uh_mx_grouped_gemm(const uint16_t* xa, int K, const int32_t* tiles, int ntiles, const uint8_t* const* w_tab,
                       const uint8_t* const* s_tab, uint16_t* out, int ldo, int N, void* stream,
                       const int* ntiles_dev, const uint8_t* const* w_tab2, const uint8_t* const* s_tab2,
                       uint16_t* out2, int max_rows);
/* mx_moe.hpp:97-99 */
int uh_mx_grouped_gemm_glu(const uint16_t* xa, int K, const int32_t* tiles, int ntiles, const uint8_t* const* w1_tab,
                           const uint8_t* const* s1_tab, const uint8_t* const* w3_tab, const uint8_t* const* s3_tab,
                           int N, const float* glu_w, const int32_t* glu_row_expert, const uint8_t* const* glu_s_tab,
                           uint16_t* glu_hh, float glu_limit, void* stream, const int* ntiles_dev);
/* No reference counterpart: the GEMV / GEMM on e4m3 activation codes q [P, K] + e8m0 qs [P, K/128]. */
int uh_mx_grouped_gemv_q(const uint8_t* q, const uint8_t* qs, int K, const int32_t* tiles, int ntiles,
                         const uint8_t* const* w_tab, const uint8_t* const* s_tab, uint16_t* out, int ldo, int N,
                         void* stream, const int* ntiles_dev, const uint8_t* const* w_tab2,
                         const uint8_t* const* s_tab2, uint16_t* out2, int max_rows, const float* glu_w,
                         const int32_t* glu_row_expert, const uint8_t* const* glu_s_tab, uint16_t* glu_hh,
                         uint8_t* glu_hq, uint8_t* glu_hs, float glu_limit);
/* No reference counterpart: uh_mx_xform_in_fp8 + uh_mx_grouped_gemv_q in one launch (the workgroup quantizes its
 * tile's token rows x[x_rows[r]] per 128 while staging them); bit-identical outputs. */
int uh_mx_grouped_gemv_x(const uint16_t* x, int ldx, const int32_t* x_rows, int K, const int32_t* tiles, int ntiles,
                         const uint8_t* const* w_tab, const uint8_t* const* s_tab, uint16_t* out, int ldo, int N,
                         void* stream, const int* ntiles_dev, const uint8_t* const* w_tab2,
                         const uint8_t* const* s_tab2, uint16_t* out2, int max_rows, const float* glu_w,
                         const int32_t* glu_row_expert, const uint8_t* const* glu_s_tab, uint16_t* glu_hh,
                         uint8_t* glu_hq, uint8_t* glu_hs, float glu_limit);
/* No reference counterpart: uh_mx_xform_in_fp8 + uh_mx_grouped_gemm_q in one launch (prefill tiles). */
int uh_mx_grouped_gemm_x(const uint16_t* x, int ldx, const int32_t* x_rows, int K, const int32_t* tiles, int ntiles,
                         const uint8_t* const* w_tab, const uint8_t* const* s_tab, uint16_t* out, int ldo, int N,
                         void* stream, const int* ntiles_dev, const uint8_t* const* w_tab2,
                         const uint8_t* const* s_tab2, uint16_t* out2, const float* glu_w,
                         const int32_t* glu_row_expert, const uint8_t* const* glu_s_tab, uint16_t* glu_hh,
                         uint8_t* glu_hq, uint8_t* glu_hs, float glu_limit);
/* No reference counterpart: the prefill GEMM (uh_mx_grouped_gemm_q, one projection) with fp32 outputs (before bf16
 * rounding), for accuracy checks. N % 256 == 0. */
int uh_mx_grouped_gemm_q_f32out(const uint8_t* q, const uint8_t* qs, int K, const int32_t* tiles, int ntiles,
                                const uint8_t* const* w_tab, const uint8_t* const* s_tab, float* out, int ldo, int N,
                                void* stream, const int* ntiles_dev);
/* No reference counterpart: the prefill GEMM's arithmetic on e4m3 codes: 1 (default) exact bf16 dequantization +
 * bf16 MFMA (the parity arithmetic), 0 the block-scaled MFMA (a speed mode outside the parity tolerance).
 * Process-wide; returns the previous setting. */
int uh_mx_gemm_set_exact(int on);
/* No reference counterpart: uh_mx_grouped_gemv_q with fp32 outputs (before bf16 rounding), for accuracy checks. */
int uh_mx_grouped_gemv_q_f32out(const uint8_t* q, const uint8_t* qs, int K, const int32_t* tiles, int ntiles,
                                const uint8_t* const* w_tab, const uint8_t* const* s_tab, float* out, int ldo, int N,
                                void* stream, const int* ntiles_dev, int max_rows);
/* No reference counterpart: the prefill GEMM on e4m3 activation codes q [P, K] + e8m0 qs [P, K/128] (the form the
 * forward uses; same arguments as uh_mx_grouped_gemv_q). */
int uh_mx_grouped_gemm_q(const uint8_t* q, const uint8_t* qs, int K, const int32_t* tiles, int ntiles,
                         const uint8_t* const* w_tab, const uint8_t* const* s_tab, uint16_t* out, int ldo, int N,
                         void* stream, const int* ntiles_dev, const uint8_t* const* w_tab2,
                         const uint8_t* const* s_tab2, uint16_t* out2, int max_rows, const float* glu_w,
                         const int32_t* glu_row_expert, const uint8_t* const* glu_s_tab, uint16_t* glu_hh,
                         uint8_t* glu_hq, uint8_t* glu_hs, float glu_limit);

/* ---- routing and dispatch (src/kernels/ref.hpp, src/kernels/moe_dispatch.hpp). plan: int32[5]
 * {P, remote0, n_local_tiles, n_remote_tiles, n_remote_tokens}. ---- */
/* ref.hpp:243-245 */
int uh_route(const float* logits, const float* bias, const int32_t* tid2eid, const int32_t* ids, int32_t* sel,
             float* weights, int T, int E, int K, float route_scale, void* stream, const float* bias_vl, int vocab);
/* ref.hpp:247-249 */
int uh_route_fast(const float* logits, const float* bias, const int32_t* tid2eid, const int32_t* ids, int32_t* sel,
                  float* weights, int T, int E, int K, float route_scale, void* stream, const float* bias_vl,
                  int vocab);
/* moe_dispatch.hip:308-356 (route_token_wave, GLM sigmoid routing) */
int uh_route_glm(const float* logits, const float* bias, int32_t* sel, float* weights, int T, int E, int K,
                 float route_scale, void* stream);
/* No reference counterpart: the synthetic workload's softmax top-K, renormalised over the picks. */
int uh_route_softmax(const float* logits, int32_t* sel, float* weights, int T, int E, int K, void* stream);
/* moe_dispatch.hpp:25: dst[i] = (uint8) sel[i], the routing trace (dst may be pinned host memory). */
int uh_moe_trace(const int32_t* sel, int n, uint8_t* dst, void* stream);
/* elem_fast.hpp:10-12, 21-22: rmsnorm of rows (any dim, out of place); the mHC post-mix of rows x [T, dim] into
 * out [T, hc, dim] from the streams res (out may be res; post [T, hc], comb [T, hc, hc], hc <= 4). */
int uh_rmsnorm_slices(const uint16_t* x, int ldx, const uint16_t* w, uint16_t* y, int ldy, int rows, int dim, float eps,
                      void* stream);
int uh_hc_post_slices(const uint16_t* x, const uint16_t* res, const float* post, const float* comb, uint16_t* out,
                      int T, int hc, int dim, void* stream);
/* moe_dispatch.hpp:26 */
int uh_moe_count(const int32_t* sel, int T, int K, int32_t* count, int E, void* stream, uint32_t* hist);
/* moe_dispatch.hpp:29-31 (resident may be NULL: all resident) */
int uh_moe_plan(int32_t* count, const uint8_t* resident, int E, int P, int32_t* plan, int32_t* local_tiles,
                int32_t* remote_tiles, int32_t* off, int32_t* fill, int max_tiles, void* stream, int tile_rows);
/* moe_dispatch.hpp:32-33 (deterministic: rows of an expert in ascending token order) */
int uh_moe_scatter(const int32_t* sel, const float* wt, int T, int K, const int32_t* off, int32_t* fill,
                   int32_t* eidx, float* ewt, int32_t* row_expert, int32_t* pidx, void* stream);
/* moe_dispatch.hpp:124 (MoeSmallArgs without the resident mask and remote-side fields; ds_* or route_* logits:
 * routing in-launch) */
int uh_moe_dispatch_small(const int32_t* sel, const float* wt, int T, int K, int E, int P, int max_tiles,
                          int tile_rows, int32_t* plan, int32_t* tiles, int32_t* eidx, float* ewt,
                          int32_t* row_expert, int32_t* pidx, uint32_t* hist, const float* route_logits,
                          const float* route_bias, float route_scale, const float* ds_logits, const float* ds_bias,
                          const float* ds_bias_vl, const int32_t* ds_tid2eid, const int32_t* ids, int vocab,
                          void* stream);
/* No reference counterpart: uh_moe_dispatch_small for local steps of up to 512 picks (T * K, e.g. T = 64 at top-6;
 * no resident mask or remote outputs), softmax_logits (may be NULL): softmax top-K routing in the launch. */
int uh_moe_dispatch_mid(const int32_t* sel, const float* wt, int T, int K, int E, int P, int max_tiles, int tile_rows,
                        int32_t* plan, int32_t* tiles, int32_t* eidx, float* ewt, int32_t* row_expert, int32_t* pidx,
                        uint32_t* hist, const float* route_logits, const float* route_bias, float route_scale,
                        const float* ds_logits, const float* ds_bias, const float* ds_bias_vl,
                        const int32_t* ds_tid2eid, const int32_t* ids, int vocab, const float* softmax_logits,
                        void* stream);
/* ref.hpp:251-252 */
int uh_swiglu(const uint16_t* gate, const uint16_t* up, const float* w, uint16_t* h, int rows, int dim, float limit,
              void* stream);
/* ref.hpp:254 */
int uh_scatter_add(const uint16_t* src, const int32_t* rows_idx, float* y, int n, int dim, void* stream);
/* ref.hpp:255 */
int uh_gather_rows(const uint16_t* src, const int32_t* rows_idx, uint16_t* dst, int n, int dim, void* stream);
/* ref.hpp:258-259 (shared may be NULL: zero) */
int uh_moe_combine(const uint16_t* pair_out, const int32_t* pidx, const uint16_t* shared, uint16_t* out, int T, int K,
                   int dim, void* stream);

/* ---- quantization and dense fp8 (src/kernels/ref.hpp, gemv.hpp, gemm_wmma.hpp) ---- */
/* ref.hpp:128 */
int uh_act_quant_fp8(const uint16_t* x, int ldx, uint8_t* q, uint8_t* s, int rows, int cols, int block, void* stream);
/* ref.hpp:130 */
int uh_fake_quant_fp8(uint16_t* x, int ldx, int rows, int cols, int block, void* stream);
/* ref.hpp:25 */
int uh_fake_quant_fp4(uint16_t* x, int ldx, int rows, int cols, int block, void* stream);
/* tools/ref/oracle/kernel.py:43-55 with scale_fmt=None (fp32 scales) */
int uh_act_quant_fp8_f32s(const uint16_t* x, int ldx, uint8_t* q, float* s, int rows, int cols, int block,
                          void* stream);
/* ref.hpp:135-136 */
int uh_gemm_w8a8(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                 int M, int N, int K, void* stream);
/* gemm_wmma.hpp:15-16 */
int uh_gemm_w8a8_wmma(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                      int M, int N, int K, void* stream);
/* gemv.hpp:23-24 */
int uh_gemv_w8a8(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                 int M, int N, int K, void* stream);
/* gemv.hpp:40-52 (GemvPart, gemv_w8a8_parts): n (1..3) column ranges on one input, given as host arrays of n
 * entries: device pointers w (e4m3 [N_i, K]), sw (e8m0 [ceil(N_i/128), K/128]), c (bf16 [M, ldc_i]); ints ldc, N. */
int uh_gemv_w8a8_parts(const uint8_t* a, const uint8_t* sa, const void* const* w, const uint8_t* const* sw,
                       void* const* c, const int* ldc, const int* N, int nparts, int M, int K, void* stream);
/* gemv.hpp:31-35, 56-57 (GemvQuant, gemv_w8a8_glu): gate / up [M, I] into gate / up, then act_quant_fp8 of
 * bf16(SwiGLU(gate, up)) into q [M, I] / qs [M, I/128]; counters [I/128] zero on entry, left zero (may be NULL). */
int uh_gemv_w8a8_glu(const uint8_t* a, const uint8_t* sa, const uint8_t* w_gate, const uint8_t* sw_gate,
                     uint16_t* gate, int ldg, const uint8_t* w_up, const uint8_t* sw_up, uint16_t* up, int ldu, int I,
                     int M, int K, float limit, uint8_t* q, uint8_t* qs, uint32_t* counters, void* stream);
/* kernel.py fp8_gemm with fp32 scales (scale_fmt=None); gemm_wmma.hip:89-100's fold */
int uh_gemm_fp8_f32s(const uint8_t* a, const float* sa, const uint8_t* w, const float* sw, uint16_t* c, int ldc,
                     int M, int N, int K, void* stream);
/* ---- the expert pack (src/model/expert_pack.hpp:1-92; the file format byte for byte) ---- */
/* XXH64 of len bytes (a value, not a status). */
uint64_t uh_pack_xxh64(const void* data, size_t len, uint64_t seed);
/* The writer (tools/expert_pack's job, from host arrays): (n_layers + n_mtp) * n_experts slots; parts: host table of
 * 6 pointers per slot {w1 codes [w13_out, w13_in/2], w1 scales [w13_out, w13_in/32], w3 ..., w2 codes
 * [w2_out, w2_in/2], w2 scales}, row-major, or six NULLs for an absent slot. */
int uh_pack_write(const char* path, int n_layers, int n_mtp, int n_experts, int w13_out, int w13_in, int w2_out,
                  int w2_in, const uint8_t* const* parts, uint64_t config_hash, uint64_t source_hash);
/* expert_pack.hpp:88-89 (read_header): the validated header's 264 bytes into header (host). */
int uh_pack_read_header(const char* path, uint8_t* header);
/* The loader: slots [first, first + count) into device memory dst + i * stride (stride >= slot_bytes, % 256 == 0),
 * through pinned double-buffered staging; verify: each slot's xxh64 against the checksum table; direct: O_DIRECT.
 * Synchronous on stream at return. */
int uh_pack_load(const char* path, size_t first, size_t count, void* dst, size_t stride, int verify, int direct,
                 void* stream);
/* The forward's expert table (6 x E device pointers, {w1 codes, w1 scales, w3 ..., w2 scales} x E, as
 * uh_mx_moe_forward takes it) of E slots loaded at slots + e * stride, into the host array tab [6 * E]. */
int uh_pack_expert_table(const uint8_t* header, const void* slots, size_t stride, int E, uint64_t* tab);
/* elem_fast.hpp:23-26: rmsnorm of x [rows, dim] with w [dim] into y, then (q set) act_quant_fp8 (block 128) of y into
 * q [rows, dim] / qs [rows, dim / 128], one launch. *launched = 0 where the reference's returns false (in place, or
 * slices not whole multiples of 256 values): nothing was done. */
int uh_rmsnorm_quant_slices(const uint16_t* x, int ldx, const uint16_t* w, uint16_t* y, int ldy, uint8_t* q,
                            uint8_t* qs, int rows, int dim, float eps, int* launched, void* stream);
/* moe_dispatch.hpp:71-76: act_quant_fp8 (block 128) of rows x[u2t[u]] for u < plan[4] (n_remote_tokens, on the
 * device) into q [U, dim] / s [U, dim / 128]; grid for max_tokens. */
int uh_quant_remote_tokens(const uint16_t* x, int dim, const int32_t* u2t, const int32_t* plan, uint8_t* q, uint8_t* s,
                           int max_tokens, void* stream);
/* moe_dispatch.hpp:34-40, 125-126: the remote rows [plan[1], plan[0]) of src to the same rows of dst (bf16, dim % 8);
 * the plan, remote tiles and remote rows' weights / experts to the remote side's staging; weights / experts only. */
int uh_copy_remote_rows(const uint16_t* src, uint16_t* dst, const int32_t* plan, int dim, int max_rows, void* stream);
int uh_stage_remote(const int32_t* plan, const int32_t* rtiles, const float* ewt, const int32_t* row_expert,
                    int32_t* plan_dst, int32_t* tiles_dst, float* w_dst, int32_t* e_dst, int max_rows, void* stream);
int uh_copy_remote_meta(const float* ewt, const int32_t* row_expert, float* w_dst, int32_t* e_dst, const int32_t* plan,
                        int max_rows, void* stream);
/* moe_dispatch.hpp:41-46: compact remote tokens: tok2u [T], u2t [U], plan[4] = U, p2u [P] (remote rows), u2p [U, K]
 * (may be NULL). One workgroup. */
int uh_remote_tokens(const int32_t* pidx, const int32_t* eidx, int T, int K, int32_t* plan, int32_t* tok2u,
                     int32_t* u2t, int32_t* p2u, int32_t* u2p, void* stream);
/* moe_dispatch.hpp:47-52: dst [U, dim] = bf16 sums of each compact token's remote pair rows. */
int uh_remote_combine(const uint16_t* pair_out, const int32_t* u2p, const int32_t* plan, uint16_t* dst, int K, int dim,
                      int max_tokens, void* stream);
/* moe_dispatch.hpp:53-60: dst[u] = x[u2t[u]]; src [U, dim] -> rows plan[1] + u of dst. */
int uh_copy_remote_tokens(const uint16_t* x, int dim, const int32_t* u2t, const int32_t* plan, uint16_t* dst,
                          int max_tokens, void* stream);
int uh_copy_remote_partial(const uint16_t* src, uint16_t* dst, const int32_t* plan, int dim, int max_tokens,
                           void* stream);
/* moe_dispatch.hpp:61-70: out [T, dim] = bf16(local pair rows + remote partial + shared (may be NULL)); the _link form
 * reads the partial from row tok2u[t] of remote and, with hc_x set, post-mixes each output value into the streams
 * hc_x [T, hc, dim] (post [T, hc], comb [T, hc, hc], hc <= 4) in place. */
int uh_moe_combine_partial(const uint16_t* pair_out, const int32_t* pidx, const int32_t* plan, const int32_t* tok2u,
                           const uint16_t* shared, uint16_t* out, int T, int K, int dim, void* stream);
int uh_moe_combine_partial_link(const uint16_t* pair_out, const int32_t* pidx, const int32_t* plan,
                                const int32_t* tok2u, const uint16_t* remote, const uint16_t* shared, uint16_t* out,
                                int T, int K, int dim, uint16_t* hc_x, const float* post, const float* comb, int hc,
                                void* stream);
/* moe_dispatch.hpp:79-124: moe_dispatch_small with the resident mask and the remote-side fields (routing from
 * ds_logits when not NULL, else sel / wt are inputs). remote: stage plan_dst / tiles_dst / w_dst / e_dst; qin: also
 * tok2u, u2t, p2u, u2p (may be NULL), then x_dst (may be NULL) and q_dst / qs_dst (may be NULL) from x [T, dim];
 * req_flag (may be NULL) = req_value, stored last with system-scope release. */
int uh_moe_dispatch_small_remote(const int32_t* sel, const float* wt, int T, int K, int E, int P, int max_tiles,
                                 int tile_rows, int32_t* plan, int32_t* tiles, int32_t* remote_tiles, int32_t* eidx,
                                 float* ewt, int32_t* row_expert, int32_t* pidx, const uint8_t* resident,
                                 const float* ds_logits, const float* ds_bias, float route_scale, int remote, int qin,
                                 int32_t* tok2u, int32_t* u2t, int32_t* p2u, int32_t* u2p, int32_t* plan_dst,
                                 int32_t* tiles_dst, float* w_dst, int32_t* e_dst, const uint16_t* x, int dim,
                                 uint16_t* x_dst, uint8_t* q_dst, uint8_t* qs_dst, uint32_t* req_flag,
                                 uint32_t req_value, void* stream);
/* ref.hpp:42-45 (reference order), gemm_wmma.hpp:24-26 (fast path), gemv.hpp:36-37 (GEMV, M <= 32): grouped
 * "mgk,grk->mgr" with fp8 weights x 128x128 e8m0 scales. a bf16 [M, G, K], w e4m3 [G R, K],
 * sw [ceil(G R / 128), K / 128], c bf16 [M, G, R]; K % 128 == 0. uh_gemv_grouped_fp8w with q set also writes
 * act_quant_fp8 (block 128) of c into q [M, G R] / qs [M, G R / 128] ((G R) % 128 == 0; counters may be NULL). */
int uh_gemm_grouped_fp8w(const uint16_t* a, const uint8_t* w, const uint8_t* sw, uint16_t* c, int M, int G, int R,
                         int K, void* stream);
int uh_gemm_grouped_fp8w_wmma(const uint16_t* a, const uint8_t* w, const uint8_t* sw, uint16_t* c, int M, int G,
                              int R, int K, void* stream);
int uh_gemv_grouped_fp8w(const uint16_t* a, const uint8_t* w, const uint8_t* sw, uint16_t* c, int M, int G, int R,
                         int K, uint8_t* q, uint8_t* qs, uint32_t* counters, void* stream);
/* No reference counterpart: uh_act_quant_fp8_f32s (block 128) of bf16 x [M, ldx] fused into uh_gemm_fp8_f32s for
 * M <= 16 (decode rows): the same results bit for bit, one launch. */
int uh_gemm_fp8_f32s_x(const uint16_t* x, int ldx, const uint8_t* w, const float* sw, uint16_t* c, int ldc, int M,
                       int N, int K, void* stream);
/* ref.hpp:139-140 and :142-143: the reference-order (bit-exact) a8w4 GEMMs */
int uh_gemm_a8w4(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                 int M, int N, int K, void* stream);
int uh_gemm_a8w4_tiled(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                       int M, int N, int K, void* stream);
/* No reference counterpart (checkpoint-side preparation): e4m3 codes of fp32 weights [N, K] with one fp32 scale per
 * 128 x 128 block, s = max(amax, 1e-4) / 448 (fp32, times fp32(1/448)). */
int uh_quant_weight_fp8_f32s(const float* w, uint8_t* q, float* s, int N, int K, void* stream);

/* ---- the routed-expert FFN in one call (src/model/forward_ref.hip:449-474 native branch + moe_device_dispatch
 * :1052-1156 + moe_combine): router logits [T, E] -> softmax top-K -> dispatch -> xform (fp8) -> w1/w3 + SwiGLU ->
 * w2 -> combine into out [T, D]. tab: device table of 6 * E pointers {w1 codes, w1 scales, w3 codes, w3 scales,
 * w2 codes, w2 scales} x E (tile-major), the layout of the reference's exl3_ptrs(m, f, E). ws: device workspace of
 * uh_mx_moe_workspace_size bytes. sel / wt (may be NULL): the routing is also written there. Every expert the routing
 * can pick must have all six pointers: a NULL entry's rows are skipped by the GEMVs / GEMMs (the kernels' contract)
 * and their pair rows are then undefined in the combine; an engine holding only some experts uses the remote entry
 * points (uh_moe_dispatch_small_remote, uh_remote_combine, uh_moe_combine_partial_link) instead. ---- */
size_t uh_mx_moe_workspace_size(int T, int K, int E, int D, int I);
int uh_mx_moe_forward(const uint16_t* x, const float* logits, int T, int K, int E, int D, int I,
                      const uint8_t* const* tab, float limit, void* ws, size_t ws_bytes, uint16_t* out, int32_t* sel,
                      float* wt, void* stream);
/* The same with stage events (6 hipEvent_t, recorded on `stream` before routing, after routing + dispatch, after
 * the input transform, after w1/w3 + SwiGLU, after w2, after the combine; NULL entries are skipped). */
int uh_mx_moe_forward_ev(const uint16_t* x, const float* logits, int T, int K, int E, int D, int I,
                         const uint8_t* const* tab, float limit, void* ws, size_t ws_bytes, uint16_t* out, int32_t* sel,
                         float* wt, void* stream, void* const* events);

/* No reference counterpart: uh_mx_moe_forward for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). The workspace is a fixed device array of
 * uh_mx_moe_noalloc_max_bytes() bytes (8 MiB, one per GPU, held until the process ends; decode and verify batches:
 * T <= 64 at E = 256, D = 4096, I = 2048 and top-6); shapes whose uh_mx_moe_workspace_size exceeds it fail with an
 * error. No allocation happens in the call. Every call on one GPU shares that array: calls that overlap on one GPU
 * (concurrent streams, threads) race and must be serialized by the caller. */
size_t uh_mx_moe_noalloc_max_bytes(void);
int uh_mx_moe_forward_noalloc(const uint16_t* x, const float* logits, int T, int K, int E, int D, int I,
                              const uint8_t* const* tab, float limit, uint16_t* out, int32_t* sel, float* wt,
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* UNHOLY_AMD_H */
