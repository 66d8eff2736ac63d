/*
 * cv3hip — C ABI of the MI355X (gfx950) tensor-kernel backend for the
 * CosyVoice 3 NumPy runtime.
 *
 * Every entry point takes plain device pointers, int64 sizes and an optional
 * stream (NULL = the calling thread's own stream), and returns an int status
 * (CV3_OK = 0).  On failure cv3_last_error() returns a thread-local message.
 * Status codes map onto the exceptions the reference raises:
 *   CV3_EINVAL  -> ValueError      CV3_EINDEX -> IndexError
 *   CV3_EASSERT -> AssertionError  CV3_EHIP   -> RuntimeError (HIP failure)
 *
 * The reference (cv3cpu) has no FFI of its own: its kernels are the module
 * functions of cv3cpu/ops.py and cv3cpu/quant.py, which the models resolve at
 * call time.  Each entry point below names the reference function whose work it
 * replaces; the Python host package binds them with ctypes behind those same
 * function names and signatures.
 */
#ifndef CV3HIP_H
#define CV3HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cv3_stream_opaque* cv3_stream_t;

enum { CV3_OK = 0, CV3_EINVAL = 1, CV3_EINDEX = 2, CV3_EASSERT = 3, CV3_EHIP = 4, CV3_EUNSUPPORTED = 5 };

/* element / weight kinds */
enum { CV3_F32 = 0, CV3_F16 = 1 };
enum { CV3_KIND_F32 = 0, CV3_KIND_F16 = 1, CV3_KIND_Q8 = 2, CV3_KIND_Q4 = 3 };

/* activations (cv3cpu/ops.py:30-81) */
enum {
  CV3_ACT_NONE = 0,
  CV3_ACT_SILU = 1,       /* ops.silu        ops.py:30  */
  CV3_ACT_SIGMOID = 2,    /* ops.sigmoid     ops.py:34  */
  CV3_ACT_GELU_TANH = 3,  /* ops.gelu_tanh   ops.py:41  */
  CV3_ACT_GELU = 4,       /* ops.gelu        ops.py:46  */
  CV3_ACT_MISH = 5,       /* ops.mish        ops.py:63  */
  CV3_ACT_ELU = 6,        /* ops.elu         ops.py:69  (param = alpha) */
  CV3_ACT_LEAKY = 7,      /* ops.leaky_relu  ops.py:73  (param = slope) */
  CV3_ACT_TANH = 8
};

/*
 * Linear epilogue: y = residual + gate * act(rope(acc + bias))
 *   residual: [m, ld_res] or NULL (0);  gate: gate[(row / rows_per_gate) * gate_stride + col] or NULL (1).
 *   rope (multi-row GEMMs only, rope_cos non-NULL): the DiT's interleaved partial rotary (dit.py:40-54) on
 *   columns c < rope_limit with c % rope_period < rope_width, using table row (row % rope_rows) of
 *   rope_cos / rope_sin [rope_rows, rope_width].
 * `y` may alias `residual` (each element is read and written by one thread).
 */
typedef struct {
  int act;
  float act_param;
  const float* residual;
  int64_t ld_res;
  const float* gate;
  int64_t gate_stride;
  int64_t rows_per_gate;
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_rows, rope_period, rope_width, rope_limit;
} cv3_epilogue;

/* ---------------- runtime ---------------- */
const char* cv3_last_error(void);
int cv3_init(int device);
int cv3_device_info(int* cu_count, int64_t* hbm_bytes, char* arch_name, int name_len);
int cv3_malloc(void** ptr, size_t bytes); /* stream-aware caching allocator */
int cv3_free(void* ptr);    /* behind every stream the block was used on; deferred to the graph if capturing */
/* Marks a block as used on stream s too, so its free waits for s (no counterpart in the reference, whose
 * arrays are host memory: the device analogue of a tensor used on a second stream). */
int cv3_record_stream(void* ptr, cv3_stream_t s);
int cv3_empty_cache(void);
int cv3_mem_stats(size_t* in_use, size_t* cached);
int cv3_copy_h2d(void* dst, const void* src, size_t bytes, cv3_stream_t s); /* returns when done */
int cv3_copy_d2h(void* dst, const void* src, size_t bytes, cv3_stream_t s); /* returns when done */
int cv3_copy_d2d(void* dst, const void* src, size_t bytes, cv3_stream_t s); /* stream-ordered */
int cv3_fill_zero(void* dst, size_t bytes, cv3_stream_t s);                 /* kernel (graph-safe) */
int cv3_stream_create(cv3_stream_t* s);
int cv3_stream_destroy(cv3_stream_t s);
int cv3_stream_sync(cv3_stream_t s);
int cv3_device_sync(void);
int cv3_event_create(void** ev);
int cv3_event_destroy(void* ev);
int cv3_event_record(void* ev, cv3_stream_t s);
/* Work enqueued on s after this call waits for ev's last recorded point (no counterpart in the reference:
 * orders work across streams, e.g. vocoder windows run side by side). */
int cv3_stream_wait_event(cv3_stream_t s, void* ev);
int cv3_event_elapsed_ms(void* ev0, void* ev1, float* ms);
int cv3_graph_begin(cv3_stream_t s);
int cv3_graph_end(cv3_stream_t s, void** exec);
int cv3_graph_launch(void* exec, cv3_stream_t s);
int cv3_graph_destroy(void* exec);
/* Synchronises the device and releases every graph, cached or live block, per-thread stream, and every
 * stream and event from cv3_stream_create / cv3_event_create; afterwards frees and destroys are no-ops and
 * every other entry point returns CV3_EINVAL (no counterpart in the reference: called once at process exit, before the
 * HIP runtime's own teardown). */
int cv3_shutdown(void);
/* Counts of the HIP objects the library holds: streams (per-thread and created), events (created and the
 * allocator's), captured graphs and allocator blocks; all 0 after cv3_shutdown (no counterpart in the
 * reference: lets a caller check that nothing outlives the shutdown into the runtime's exit handlers). */
int cv3_live_handles(int64_t* streams, int64_t* events, int64_t* graphs, int64_t* blocks);
/* fp32 matrix-core rate probe: workgroups x 512 threads, each wave `iters` rounds of four independent
 * v_mfma_f32_32x32x2f32 on registers; *flops = the flops issued; out holds workgroups*512 floats (no
 * counterpart in the reference: the measured ceiling beside the published 157.3 TFLOP/s). */
int cv3_mfma_peak_f32(int64_t iters, int64_t workgroups, float* out, double* flops, cv3_stream_t s);

/* ---------------- host RNG (cv3cpu/torch_rng.py; host memory, host code) ---------------- */
int cv3_mt_create(uint64_t seed, void** gen);                   /* TorchMT19937.__init__  torch_rng.py:30 */
int cv3_mt_destroy(void* gen);
int cv3_mt_uniform_f32(void* gen, int64_t n, float* out_host);  /* random_float32 / rand  torch_rng.py:88,145 */
int cv3_mt_normal_f32(void* gen, int64_t n, float* out_host);   /* randn                  torch_rng.py:117 */

/* ---------------- quantisation (cv3cpu/quant.py) ---------------- */
/* quantize_q8 (quant.py:56-67): q [n, kp] int8, scales [n, kp/block] f16 (reference) or f32
 * (per-output-channel layout: block = k).  kp = ceil(k / block) * block.  Bit-exact. */
int cv3_quantize_q8(const float* w, int64_t n, int64_t k, int64_t block, int scale_dtype, int8_t* q,
                    void* scales, cv3_stream_t s);
/* quantize_q4 (quant.py:70-86): q [n, kp/2] packed nibbles, scales [n, kp/block] f16. */
int cv3_quantize_q4(const float* w, int64_t n, int64_t k, int64_t block, uint8_t* q, void* scales_f16,
                    cv3_stream_t s);
/* QTensor.dequant_rows (quant.py:110-133): out[r - r0, :k] (row stride ld_out). */
int cv3_dequant_rows(int kind, const void* q, const void* scales, int scale_dtype, int64_t kp, int64_t block,
                     int64_t k, int64_t r0, int64_t r1, float* out, int64_t ld_out, cv3_stream_t s);
/* ops.embedding (ops.py:126-144): out[i] = table[ids[i]] (f32/f16 rows or dequantised q8/q4 rows).
 * ids are device int64; out-of-range ids return CV3_EINDEX. */
int cv3_embedding(int kind, const void* table, const void* scales, int scale_dtype, int64_t rows, int64_t cols,
                  int64_t kp, int64_t block, const int64_t* ids, int64_t n, float* out, cv3_stream_t s);

/* ---------------- linear (ops.linear ops.py:121 / quant.qmatmul quant.py:156-204) ---------------- */
/* y[m, n] = epi(x[m, :k] . w[n, :k]).  fp32 weights [n, ldw].  Small m runs a GEMV, large m the MFMA GEMM. */
int cv3_linear_f32(const float* x, int64_t m, int64_t k, int64_t ldx, const float* w, int64_t ldw, int64_t n,
                   const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi, cv3_stream_t s);
/* The fp32 linear on the bfloat16 matrix cores (ops.linear, ops.py:121-123; no separate
 * reference function): w is first split once into three bfloat16 planes [3][n][ldp] (uint16
 * bit patterns, w = hi + mid + lo to all 24 bits), then each product runs as the six plane
 * products that carry float32 precision.  K % 8 (split) and K % 64 (linear), 16-byte aligned rows. */
int cv3_split_x3(const float* w, int64_t n, int64_t k, int64_t ldw, uint16_t* planes, int64_t ldp, cv3_stream_t s);
int cv3_linear_x3(const float* x, int64_t m, int64_t k, int64_t ldx, const uint16_t* planes, int64_t ldp, int64_t n,
                  const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi, cv3_stream_t s);
/* The same linear with the weight's planes packed once in the matrix cores' fragment order:
 * frag[p][nb][t][l] (8 bfloat16) = plane p of w[32 nb + l % 32][16 t + 8 (l / 32) .. + 7], rows past n zero,
 * cv3_x3_frag_elems(n, k) uint16 in all (3 planes of ceil(n / 32) * 32 * k).  The product then loads each
 * wave's weight fragments straight into registers and stages only the activation in LDS; it returns the
 * same bits as cv3_linear_x3 on the same weight.  K % 64 == 0, 16-byte aligned rows. */
int cv3_split_x3_frag(const float* w, int64_t n, int64_t k, int64_t ldw, uint16_t* frag, cv3_stream_t s);
int cv3_x3_frag_elems(int64_t n, int64_t k, int64_t* elems);
int cv3_linear_x3_frag(const float* x, int64_t m, int64_t k, int64_t ldx, const uint16_t* frag, int64_t n,
                       const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi, cv3_stream_t s);
/* quant.qmatmul on q8 weights (quant.py:165-190) on the bfloat16 matrix cores: the activation as
 * bfloat16 planes, each int8 code exact in bfloat16 (three products per code), the block scale
 * applied to each block's sum.  K % 64 == 0, block % 64 == 0 (per-channel: block = kp). */
int cv3_linear_q8_x3(const float* x, int64_t m, int64_t k, int64_t ldx, const int8_t* q, const void* scales,
                     int scale_dtype, int64_t kp, int64_t block, int64_t n, const float* bias, float* y, int64_t ldy,
                     const cv3_epilogue* epi, cv3_stream_t s);
/* The same q8 linear with the codes packed once in fragment order: frag[nb][t][l] = the 8 codes
 * q[32 nb + l % 32][16 t + 8 (l / 32) .. + 7], rows past n zero (ceil(n / 32) * 32 * k bytes); the scales
 * stay [n, kp / block].  Each wave loads its codes straight into registers; the same bits as
 * cv3_linear_q8_x3.  K % 64 == 0 (the packed k), block % 64 == 0. */
int cv3_pack_q8_frag(const int8_t* q, int64_t n, int64_t k, int64_t ldq, int8_t* frag, cv3_stream_t s);
int cv3_linear_q8_x3_frag(const float* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qfrag, const void* scales,
                          int scale_dtype, int64_t kp, int64_t block, int64_t n, const float* bias, float* y,
                          int64_t ldy, const cv3_epilogue* epi, cv3_stream_t s);
/* quant.qmatmul on q8 weights with per-channel scales (quant.py:165-190) on the int8 matrix cores:
 * each activation row rounded once to X = rint(x 2^(30 - E)) (E the exponent of the row's largest
 * |x|) and split into its four bytes as int8 digit planes, each plane times the codes an exact
 * int32 sum, the four combined in float64, times 2^(E - 30) and the output column's scale: the dot
 * product of the codes with x rounded 30 bits below the row's largest element.  The codes packed
 * once by cv3_pack_q8_frag32: frag[nb][t][l] = the 16 codes q[32 nb + l % 32][32 t + 16 (l / 32) .. + 15],
 * rows past n zero, then each row's code sum as int32 (npad = ceil(n / 32) * 32: npad * k + 4 npad
 * bytes); scales [n].  row_exp: m int32, the rows' exponents, computed here into it (row_exp_given
 * = 0) or already there (row_exp_given = 1: cv3_layer_norm_rexp wrote them for this x).  K % 64 == 0,
 * K <= 2048, 16-byte aligned rows. */
int cv3_pack_q8_frag32(const int8_t* q, int64_t n, int64_t k, int64_t ldq, int8_t* frag, cv3_stream_t s);
int cv3_linear_q8_digits(const float* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qfrag32, const void* scales,
                         int scale_dtype, int64_t n, const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi,
                         int32_t* row_exp, int row_exp_given,
                         cv3_stream_t s);
/* Quantised weights (q8: q [n, kp] int8; q4: q [n, kp/2]); scales [n, kp/block] (f16 or f32). */
int cv3_linear_q(int kind, const float* x, int64_t m, int64_t k, int64_t ldx, const void* q, const void* scales,
                 int scale_dtype, int64_t kp, int64_t block, int64_t n, const float* bias, float* y, int64_t ldy,
                 const cv3_epilogue* epi, cv3_stream_t s);


/* ---------------- elementwise / reductions ---------------- */
/* ops.silu/sigmoid/gelu_tanh/gelu/mish/elu/leaky_relu (ops.py:30-74): y = act(x), param = alpha/slope */
int cv3_act(int act, float param, const float* x, float* y, int64_t n, cv3_stream_t s);
/* op 0: a+b, 1: a*b, 2: silu(a)*b (qwen2.py:177), 3: alpha*a + beta*b, 4: (a+b)/alpha (hift.py:165) */
int cv3_binary(int op, const float* a, const float* b, float* y, int64_t n, float alpha, float beta, cv3_stream_t s);
/* ops.snake (ops.py:77-81) over (C, T) with per-channel alpha */
int cv3_snake(const float* x, const float* alpha, float* y, int64_t c, int64_t t, float eps, cv3_stream_t s);
/* the same Snake on channels-last (t, c) data (the HiFT stack's layout, hift.py:120) */
int cv3_snake_cl(const float* x, const float* alpha, float* y, int64_t t, int64_t c, float eps, cv3_stream_t s);
/* ops.softmax / ops.log_softmax over the last axis (ops.py:84-93) */
int cv3_softmax_rows(const float* x, float* y, int64_t rows, int64_t cols, int log_softmax, cv3_stream_t s);
/* ops.rms_norm (ops.py:101-104) */
int cv3_rms_norm(const float* x, const float* w, float* y, int64_t rows, int64_t cols, float eps, cv3_stream_t s);
/* ops.layer_norm (ops.py:107-118) with optional affine (w, b) and/or the DiT AdaLN modulation
 * y = LN(x) * (1 + scale[g]) + shift[g], g = row / rows_per_group (dit.py:168-169,178). */
int cv3_layer_norm(const float* x, float* y, int64_t rows, int64_t cols, float eps, const float* w, const float* b,
                   const float* shift, const float* scale, int64_t mod_stride, int64_t rows_per_group,
                   cv3_stream_t s);
/* cv3_layer_norm that also writes each row's binary exponent row_exp[r] = max(e, -96), e the
 * frexp exponent of the row's largest |y| (0 for an all-zero row): the row scale
 * cv3_linear_q8_digits rounds to, handed to it with row_exp_given = 1.  Rows of at most 1024
 * columns, 16-byte aligned (else CV3_EUNSUPPORTED).  No counterpart in the reference: it fuses
 * the pass the digit-plane GEMM needs into the norm that feeds the GEMM (dit.py:168-169,178). */
int cv3_layer_norm_rexp(const float* x, float* y, int64_t rows, int64_t cols, float eps, const float* w,
                        const float* b, const float* shift, const float* scale, int64_t mod_stride,
                        int64_t rows_per_group, int32_t* row_exp, cv3_stream_t s);
/* rotary tables: kind 0 = DiT rope_freqs + fp32 cos/sin (dit.py:21-29,51-52); kind 1 = Qwen2 RopeCache (qwen2.py:46-56).
 * cos/sin [n, dim] for positions pos0 .. pos0+n-1. */
int cv3_rope_table(int kind, double theta, int dim, int64_t n, int64_t pos0, float* cos_out, float* sin_out,
                   cv3_stream_t s);
/* dit.apply_partial_rope (dit.py:40-54), in place on the first `rot` channels of each row */
int cv3_rope_pairs(float* x, int64_t ld, int64_t rows, int64_t rows_per_batch, int rot, const float* cos_tab,
                   const float* sin_tab, cv3_stream_t s);
/* qwen2.apply_rope (qwen2.py:64-71), in place; vector v at x + (v/per_pos)*ld_pos + (v%per_pos)*d, position pos0 + v/per_pos */
int cv3_rope_half(float* x, int64_t nvec, int64_t per_pos, int64_t ld_pos, int d, const float* cos_tab,
                  const float* sin_tab, int64_t pos0, cv3_stream_t s);
/* Flow.solve_euler CFG combine + Euler update (flow.py:86-87): x += dt * ((1 + w) d_cond - w d_uncond) */
int cv3_cfg_euler(float* x, const float* d_cond, const float* d_uncond, int64_t n, float dt, float w, cv3_stream_t s);
/* ops.interpolate_nearest (ops.py:335-336) and ops.interpolate_linear (ops.py:318-332) over (C, T) */
int cv3_interp_nearest(const float* x, float* y, int64_t c, int64_t t, int r, cv3_stream_t s);
int cv3_interp_linear(const float* x, float* y, int64_t c, int64_t t, int64_t size, int align_corners, cv3_stream_t s);
/* ops.hann_window (ops.py:339-343) */
int cv3_hann_window(int n, int periodic, float* out, cv3_stream_t s);
/* batched (rows, cols) -> (cols, rows) transpose (the reference's swapaxes/ascontiguousarray copies) */
int cv3_transpose(const float* x, float* y, int64_t batch, int64_t rows, int64_t cols, cv3_stream_t s);
/* y[i, j, l] = x[i, j, l] over a (d0, d1, d2) box, each side with its own element strides {s0, s1, s2}
 * (the DiT's [B, 80, T] <-> [B, T, 80] swaps and channel concat, dit.py:96,151-153,180) */
int cv3_copy_strided(const float* x, float* y, int64_t d0, int64_t d1, int64_t d2, const int64_t* x_strides,
                     const int64_t* y_strides, cv3_stream_t s);

/* ---------------- attention (ops.sdpa ops.py:267-300) ---------------- */
/* q (b, h, n, d), k/v (b, hk, m, d), out (b, h, n, d), each addressed by {batch, head, row} strides in floats
 * with d contiguous.  mask_kind 0 none, 1 ("causal", a), 2 ("chunk", a, b) (ops.py:244-264). */
int cv3_attention(const float* q, const float* k, const float* v, float* out, int64_t batch, int h, int hk,
                  int64_t n, int64_t m, int d, const int64_t* q_strides, const int64_t* k_strides,
                  const int64_t* v_strides, const int64_t* o_strides, float scale, int mask_kind, int64_t mask_a,
                  int64_t mask_b, cv3_stream_t s);
/* The same sdpa with head dim 64 on the bfloat16 matrix cores: q, k, v and the probabilities as three
 * bfloat16 planes each, every product as the six plane products that carry float32 precision.
 * Other head dims run the generic float32 kernel. */
int cv3_attention_x3(const float* q, const float* k, const float* v, float* out, int64_t batch, int h, int hk,
                     int64_t n, int64_t m, int d, const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides, float scale, int mask_kind,
                     int64_t mask_a, int64_t mask_b, cv3_stream_t s);

/* ---------------- convolution (ops.conv1d ops.py:165-219, ops.depthwise_conv1d ops.py:222-237) ---------------- */
/* x (cin, t_in) with strides (x_cs, x_ts), optionally nearest-upsampled by `up` before padding;
 * w (cout, cin/groups, k) contiguous; y (cout, t_out) with strides (y_cs, y_ts).
 * Epilogue: snake(acc + bias) if snake_alpha, else act(acc + bias); then + residual (strides r_cs, r_ts).
 * *t_out_ptr receives t_out; pass y = NULL to query it. */
int cv3_conv1d(const float* x, int64_t cin, int64_t t_in, int64_t x_cs, int64_t x_ts, const float* w, int64_t cout,
               int64_t k, const float* bias, int64_t stride, int64_t dilation, int64_t groups, int64_t pad_l,
               int64_t pad_r, int64_t up, float* y, int64_t y_cs, int64_t y_ts, int64_t* t_out_ptr, int act,
               float act_param, const float* snake_alpha, float snake_eps, const float* residual, int64_t r_cs,
               int64_t r_ts, cv3_stream_t s);
/* ops.conv1d (ops.py:165-219) for stride 1 and groups 1, the HiFT convs (hift.py:112-163): as cv3_conv1d, with
 * W (cout, cin, k) repacked as w_packed (cout, k, cin) and x time-contiguous (x_ts == 1); output length
 * t_in*up + pad_l + pad_r - dilation*(k-1).  Needs cin % 64 == 0 (else CV3_EUNSUPPORTED).  ksplit > 1 splits
 * the k*cin/32 reduction stages into ksplit even slices for small grids: partial sums go to `workspace`
 * (>= ksplit*cout*t_out floats) and are added in slice order before the epilogue (deterministic). */
int cv3_conv1d_packed(const float* x, int64_t cin, int64_t t_in, int64_t x_cs, const float* w_packed, int64_t cout,
                      int64_t k, const float* bias, int64_t dilation, int64_t pad_l, int64_t pad_r, int64_t up,
                      float* y, int64_t y_cs, int64_t y_ts, int act, float act_param, const float* snake_alpha,
                      float snake_eps, const float* residual, int64_t r_cs, int64_t r_ts, int64_t ksplit,
                      float* workspace, int64_t workspace_floats, cv3_stream_t s);
/* ops.conv1d (ops.py:165-219) for stride 1 and groups 1 on channels-last activations (the HiFT stack,
 * hift.py:112-163): x [t_in, ldx] (cin channels), W (cout, cin, k) repacked as w_packed (cout, k, cin),
 * y[t * y_ts + co * y_cs]; nearest upsample by `up` before the (pad_l, pad_r) zero padding; output length
 * t_in*up + pad_l + pad_r - dilation*(k-1).  Epilogue and split-K as cv3_conv1d_packed (workspace >=
 * ksplit*cout*t_out floats; ksplit divides k*cin/32).  Needs cin % 32 == 0 and 16-byte aligned rows. */
int cv3_conv1d_cl_packed(const float* x, int64_t t_in, int64_t cin, int64_t ldx, const float* w_packed,
                         int64_t cout, int64_t k, const float* bias, int64_t dilation, int64_t pad_l, int64_t pad_r,
                         int64_t up, float* y, int64_t y_ts, int64_t y_cs, int act, float act_param,
                         const float* snake_alpha, float snake_eps, const float* residual, int64_t r_ts, int64_t r_cs,
                         int64_t ksplit, float* workspace, int64_t workspace_floats, cv3_stream_t s);
/* cv3_conv1d_cl_packed on the bfloat16 matrix cores: x split into three bfloat16 planes in the
 * kernel, the packed weight given as its planes [3][cout][k * cin] (cv3_split_x3 over the packed
 * (cout, k * cin) rows), six plane products per product with float32 accumulation.  Needs an even
 * number of 32-channel stages per K slice (k * cin / 32 / ksplit). */
int cv3_conv1d_cl_packed_x3(const float* x, int64_t t_in, int64_t cin, int64_t ldx, const uint16_t* w_planes,
                            int64_t cout, int64_t k, const float* bias, int64_t dilation, int64_t pad_l,
                            int64_t pad_r, int64_t up, float* y, int64_t y_ts, int64_t y_cs, int act, float act_param,
                            const float* snake_alpha, float snake_eps, const float* residual, int64_t r_ts,
                            int64_t r_cs, int64_t ksplit, float* workspace, int64_t workspace_floats,
                            cv3_stream_t s);
/* cv3_conv1d_cl_packed_x3 with the weight planes in MFMA fragment order: w_frag is
 * cv3_split_x3_frag over the packed (cout, k * cin) rows (cv3_x3_frag_elems(cout, k * cin) elements),
 * so each wave loads its weight operands straight into registers; the same results, bit for bit.
 * Same requirements, and k * cin % 64 == 0 for the packing. */
int cv3_conv1d_cl_packed_x3f(const float* x, int64_t t_in, int64_t cin, int64_t ldx, const uint16_t* w_frag,
                             int64_t cout, int64_t k, const float* bias, int64_t dilation, int64_t pad_l,
                             int64_t pad_r, int64_t up, float* y, int64_t y_ts, int64_t y_cs, int act,
                             float act_param, const float* snake_alpha, float snake_eps, const float* residual,
                             int64_t r_ts, int64_t r_cs, int64_t ksplit, float* workspace, int64_t workspace_floats,
                             cv3_stream_t s);
/* The DiT's grouped causal conv_pos (dit.py:99-112, ops.conv1d with groups) on channels-last activations:
 * x [batch, t, ldx] (cin channels), y [batch, t, ldy] (cout channels),
 * y[b, s, co] = epi(bias[co] + sum_{j<k, c<cin/groups} W[co, c, j] x[b, s + j - pad_l, g*cin/groups + c]),
 * g = co / (cout/groups), zero outside [0, t); output length t (pad_r = k - 1 - pad_l).  w_packed is W
 * (cout, cin/groups, k) repacked as (cout, k, cin/groups).  Needs 64 output channels per group,
 * cin/groups % 32 == 0 and k*cin/groups % 64 == 0 (else CV3_EUNSUPPORTED); epilogue as for linears. */
int cv3_conv1d_cl(const float* x, int64_t batch, int64_t t, int64_t cin, int64_t ldx, const float* w_packed,
                  int64_t cout, int64_t k, int64_t groups, int64_t pad_l, const float* bias, float* y, int64_t ldy,
                  const cv3_epilogue* epi, cv3_stream_t s);
/* cv3_conv1d_cl on the bfloat16 matrix cores: w_frag is the packed (cout, k, cin/groups) weight as bfloat16
 * planes in fragment order (cv3_split_x3_frag with n = cout, k = k * cin/groups; cv3_x3_frag_elems elements), six
 * plane products per product with float32 accumulation.  Same requirements, and k * cin/groups % 64 == 0. */
int cv3_conv1d_cl_x3f(const float* x, int64_t batch, int64_t t, int64_t cin, int64_t ldx, const uint16_t* w_frag,
                      int64_t cout, int64_t k, int64_t groups, int64_t pad_l, const float* bias, float* y, int64_t ldy,
                      const cv3_epilogue* epi, cv3_stream_t s);
int cv3_depthwise_conv1d(const float* x, int64_t c, int64_t t_in, const float* w, int64_t k, const float* bias,
                         int64_t dilation, int64_t pad_l, int64_t pad_r, float* y, int64_t* t_out_ptr,
                         cv3_stream_t s);

/* ---------------- STFT (ops.stft ops.py:346-355, ops.istft ops.py:358-377, hift.decode hift.py:204-210) ---------------- */
/* re/im planes (n_fft/2+1, frames); *frames_ptr receives the frame count (re = NULL to query). */
int cv3_stft(const float* x, int64_t n, int n_fft, int hop, const float* win, int center, float* re, float* im,
             int64_t* frames_ptr, cv3_stream_t s);
/* mode 0: spectrum (re, im) planes; mode 1: HiFT head from conv_post's (log-magnitude, phase) planes with a
 * +-limit clip.  frame_buf: frames * n_fft floats of caller scratch. */
int cv3_istft(int mode, const float* a, const float* b, int64_t frames, int n_fft, int hop, const float* win,
              int center, int64_t length, float limit, float* frame_buf, float* y, int64_t* out_len_ptr,
              cv3_stream_t s);

/* ---------------- HiFT source (cv3cpu/models/hift.py:56-111, 212-218) ---------------- */
/* F0 classifier on the condnet output x (c, t) at strides (x_cs, x_ts): f0[t] = float32(|sum_c x w + b|), summed
 * in float64 (hift.py:69-72 with inference()'s float32 cast, hift.py:216). */
int cv3_f0_classify(const float* x, int64_t c, int64_t t, int64_t x_cs, int64_t x_ts, const float* w, const float* b,
                    float* f0, cv3_stream_t s);
/* HiFTGenerator.excitation (hift.py:90-111): float32 f0 [t] -> merged source [up * t].  noise [up * t, harmonics]
 * is the dither buffer (hift.py:75-81), l_w [harmonics] / l_b [1] the m_source.l_linear weights; phase is
 * t * harmonics doubles of caller scratch.  harmonics <= 16. */
int cv3_nsf_source(const float* f0, int64_t t, int up, int harmonics, double sampling_rate, double alpha, double sigma,
                   double voiced_threshold, const float* noise, const float* l_w, const float* l_b, double* phase,
                   float* out, cv3_stream_t s);

/* ---------------- Qwen2 decode step (cv3cpu/models/qwen2.py:139-179, cv3cpu/models/llm.py:68-77,112-123) --------- */
/* One stacked quantised weight: `rows` rows per layer, layer l row r at q + (l * rows + r) * row_bytes, its
 * scales at scales + (l * rows + r) * (kp / block).  kind CV3_KIND_Q8: int8 codes, row_bytes = kp, kp and
 * block multiples of 16; per-output-channel is block = kp with float32 scales, the reference's q8
 * (quant.py:56-67) block = 64 with float16 scales.  kind CV3_KIND_Q4: the reference's packed nibbles
 * (quant.py:70-86, block 32, +8 bias, float16 scales), row_bytes = kp / 2, kp and block multiples of 32. */
typedef struct {
  const void* q;
  const void* scales;
  int64_t rows, k, kp, block;
  int scale_dtype; /* CV3_F32 or CV3_F16 */
  int kind;        /* CV3_KIND_Q8 or CV3_KIND_Q4 */
} cv3_qweight;

/* Device pointers of a resident Qwen2 body + CosyVoice3 LM head.  qkv stacks [q; k; v] rows per layer
 * (heads*dh + 2*kv_heads*dh), gate_up stacks [gate; up] (2*inter); qkv_bias [layers, qkv rows];
 * ln1 / ln2 [layers, hidden]; norm [hidden]; head = llm_decoder [vocab, hidden] with head_bias (may be
 * NULL); embedding = speech_embedding [vocab, hidden] (q8); rope_cos / rope_sin [cap, head_dim] from
 * RopeCache (qwen2.py:35-61). */
typedef struct {
  int64_t layers, hidden, heads, kv_heads, head_dim, inter;
  float eps;
  cv3_qweight qkv, o, gate_up, down, head, embedding;
  const float* qkv_bias;
  const float* ln1;
  const float* ln2;
  const float* norm;
  const float* head_bias;
  const float* rope_cos;
  const float* rope_sin;
} cv3_qwen2_model;

/* Device state of one decode stream.  k_cache / v_cache [layers, kv_heads, cap, head_dim] (the KVCache of
 * qwen2.py:74-121); pos = position of the current input token; token = last selected id; history [cap]
 * receives each selected id at its input position; x [hidden] is the residual stream and holds the
 * current input embedding between steps; logits [vocab]; workspace of at least
 * 1024 + heads*16*64 + heads*16*2 + inter + 64 floats.
 * cap <= 1024, heads <= 16, head_dim <= 64. */
typedef struct {
  float* k_cache;
  float* v_cache;
  int64_t cap;
  int64_t* pos;
  int64_t* token;
  int64_t* history;
  float* x;
  float* logits;
  float* workspace;
  int64_t workspace_floats;
} cv3_qwen2_state;

/* One greedy token: Qwen2Model.forward on x at position pos (qwen2.py:139-179), llm_decoder head
 * (llm.py:74-77), argmax with ties to the lowest id (the stable argsort of llm.py:138), then
 * x = speech_embedding[id] (llm.py:121), history[pos + 1] = id, pos += 1.  Reads pos from device
 * memory, so one captured graph of this call serves every step.  The caller keeps pos + 1 < cap. */
int cv3_qwen2_decode_step(const cv3_qwen2_model* m, const cv3_qwen2_state* s, cv3_stream_t stream);
/* cv3_qwen2_decode_step without a caller workspace, for callers that cannot allocate (code under HIP graph
 * capture, serving loops that forbid hipMalloc): no counterpart in the reference.  s->workspace and
 * s->workspace_floats are ignored; the step's scratch is a fixed device array of the library (137.5 KB, held
 * on each device until the process ends), so it allocates nothing.  Geometries beyond that scratch (more than
 * 16 heads, or an intermediate size above 16384) are rejected.  Every call on one device shares the array, so
 * the library orders them: a call from another stream than the previous call's waits for that call's end (an
 * event created once per device by cv3_init).  Under graph capture nothing is recorded: the captured steps share
 * the array, and replays of graphs holding them must not overlap on one device. */
int cv3_qwen2_decode_step_noalloc(const cv3_qwen2_model* m, const cv3_qwen2_state* s, cv3_stream_t stream);
/* The decode step's q8 / q4 GEMV on its own (quant.py:172-204 at m = 1, K1): layer `layer` of a stacked weight,
 * y = W . v with v = x, or v = rms_norm(x, rms_w, eps) when rms_w is given (ops.py:101-104).
 * mode 0: y = W v + bias (bias may be NULL); 1: y += W v; 2: rows are [gate; up] (rows/2 each) and
 * y = silu(gate . v) * (up . v) (qwen2.py:175-177).  K <= 16384 (mode 2: K <= 5120). */
int cv3_gemv_q8(const cv3_qweight* w, int64_t layer, const float* x, const float* rms_w, float eps, const float* bias,
                float* y, int mode, cv3_stream_t stream);
/* The sampler of CosyVoice3LM (llm.py:37-49 nucleus_sampling, llm.py:125-149 _sample) for a decode step.
 * ctl is 6 int64 of device memory: [0] the position of the generation's first input, [1] 0 while running, set to
 * (step + 1) when a stop id (speech_token_size .. +199) is drawn, after which steps leave the state untouched;
 * [2..5] NumPy's PCG64 state (state high, low, increment high, low 64 bits), advanced by the draws the reference
 * takes (one per token, two when the repetition test resamples).  rep_threshold = win_size * tau_r, formed in
 * double as the reference compares it; steps below min_len mask the eos id (every stop id with strict_min_len).
 * top_k 1..64, vocabulary <= 8192. */
typedef struct {
  double top_p;
  double rep_threshold;
  int64_t top_k;
  int64_t win_size;
  int64_t speech_token_size;
  int64_t min_len;
  int strict_min_len;
  int64_t* ctl;
} cv3_sampler;
/* cv3_qwen2_decode_step with the token drawn by the sampler instead of the argmax (llm.py:112-123). */
int cv3_qwen2_decode_step_sampled(const cv3_qwen2_model* m, const cv3_qwen2_state* s, const cv3_sampler* smp,
                                  cv3_stream_t stream);
/* The decode step of cv3_qwen2_decode_step (Qwen2Model.forward, qwen2.py:139-179; llm_decoder, llm.py:74-77;
 * the argmax and next input, llm.py:121,138) as ONE kernel launch (q8 weights, head dim 64, cache <= 1024
 * positions): one workgroup per CU runs every layer; vectors crossing workgroups travel as (epoch, value) words
 * in `words` (device memory of *words uint64 from cv3_qwen2_persist_words; zeroed at allocation, then whatever
 * earlier launches left), with every wait bounded: a word that never arrives sets *err (device int64, caller
 * clears it) and the launch ends early, its results invalid.  epoch_base must differ between launches (count
 * launches, times 256, never 0; clear `words` when the count wraps).  select 1: the greedy pick and bookkeeping
 * of cv3_qwen2_decode_step; select 0: logits only (then cv3_qwen2_select).  The workgroups must all be resident
 * at once: cooperative 1 launches with hipLaunchCooperativeKernel, which guarantees that or fails; cooperative 0
 * launches ordinarily (about 20 us less per token), for a device with nothing else running: a workgroup that
 * cannot start shows up as *err, not as a hang.  One such launch at a time per device.  With one scale
 * per [gate; up] row (the per-channel profile) the MLP's [gate; up] dot products run as exact int8 MFMAs on
 * base-128 digit planes of the normed activation; results stay within the same 1e-5 of the oracle. */
typedef struct {
  uint64_t* words;
  int64_t words_len;
  int64_t* err;
  uint32_t epoch_base;
  int workgroups;  /* 0: one per CU, at most 256 */
  int cooperative; /* 1: hipLaunchCooperativeKernel; 0: ordinary launch */
} cv3_persist;
int cv3_qwen2_persist_words(const cv3_qwen2_model* m, int workgroups, int64_t* words);
int cv3_qwen2_decode_step_persistent(const cv3_qwen2_model* m, const cv3_qwen2_state* s, const cv3_persist* p,
                                     int select, cv3_stream_t stream);
/* The token selection of a decode step alone, on the logits already in s->logits: greedy (smp == NULL) or the
 * sampler; then x = speech_embedding[id], history[pos + 1] = id, pos += 1.  After a prompt prefill that left the
 * last position's logits and pos = that position, this draws the first speech token (llm.py:112-121, i = 0). */
int cv3_qwen2_select(const cv3_qwen2_model* m, const cv3_qwen2_state* s, const cv3_sampler* smp, cv3_stream_t stream);
/* n doubles of Generator.random() from the PCG64 state pcg[0..3] (device, layout as in cv3_sampler.ctl[2..5]),
 * which is advanced: the draw primitive of the sampler, exposed so its stream can be checked against NumPy. */
int cv3_pcg64_random(int64_t* pcg, int64_t n, double* out, cv3_stream_t stream);
/* x = speech_embedding[*token] (ops.py:126-144): the first input of a decode. */
int cv3_qwen2_embed_token(const cv3_qwen2_model* m, const cv3_qwen2_state* s, cv3_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CV3HIP_H */
