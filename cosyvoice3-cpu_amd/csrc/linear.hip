// ops.linear / quant.qmatmul entry points (cv3cpu/ops.py:121-123,
// cv3cpu/quant.py:156-204): GEMV for up to four activation rows, the MFMA GEMM
// above that (fp32, q8 and q4 weights alike).
#include "common.hpp"

namespace cv3 {
int gemv(int wk, bool sf16, bool swiglu, const float* x, int64_t m, int64_t k, int64_t ldx, const void* w,
         int64_t ldw_bytes, const void* scales, int64_t nb, int64_t block, int64_t n, const float* bias, float* y,
         int64_t ldy, const cv3_epilogue* epi, const float* rms_w, float rms_eps, hipStream_t st);
// bkind: 0 fp32, 1 q8, 2 q4 weights
int gemm(int bkind, const float* a, int64_t m, int64_t k, int64_t lda, const void* b, int64_t ldb,
         const void* scales, bool sf16, int64_t nb, int64_t block, int64_t n, const float* bias, float* c,
         int64_t ldc, const cv3_epilogue* epi, hipStream_t st);
int gemm_x3(const float* a, int64_t m, int64_t k, int64_t lda, const uint16_t* planes, int64_t ldp, int64_t pstride,
            int64_t n, const float* bias, float* c, int64_t ldc, const cv3_epilogue* epi, hipStream_t st);
int split_x3(const float* w, int64_t n, int64_t k, int64_t ldw, uint16_t* planes, int64_t ldp, int64_t pstride,
             hipStream_t st);
int64_t x3_frag_plane(int64_t n, int64_t k);
int split_x3_frag(const float* w, int64_t n, int64_t k, int64_t ldw, uint16_t* frag, hipStream_t st);
int gemm_x3f(const float* a, int64_t m, int64_t k, int64_t lda, const uint16_t* frag, int64_t n, const float* bias,
             float* c, int64_t ldc, const cv3_epilogue* epi, hipStream_t st);
int pack_q8_frag(const int8_t* q, int64_t n, int64_t k, int64_t ldq, int8_t* frag, hipStream_t st);
int pack_q8_frag32(const int8_t* q, int64_t n, int64_t k, int64_t ldq, int8_t* frag, hipStream_t st);
int gemm_q8d(const float* a, int64_t m, int64_t k, int64_t lda, const int8_t* qfrag32, const void* scales, bool sf16,
             int64_t n, const float* bias, float* c, int64_t ldc, const cv3_epilogue* epi, int* rexp, bool rexp_given, hipStream_t st);
int gemm_x3qf(const float* a, int64_t m, int64_t k, int64_t lda, const int8_t* qfrag, const void* scales, bool sf16,
              int64_t nb, int64_t block, int64_t n, const float* bias, float* c, int64_t ldc,
              const cv3_epilogue* epi, hipStream_t st);
int gemm_x3q(const float* a, int64_t m, int64_t k, int64_t lda, const int8_t* q, int64_t ldq, const void* scales,
             bool sf16, int64_t nb, int64_t block, int64_t n, const float* bias, float* c, int64_t ldc,
             const cv3_epilogue* epi, hipStream_t st);
}  // namespace cv3

using namespace cv3;

static constexpr int64_t kGemvRows = 4;  // quant.py:43 THREAD_ROW_LIMIT: the decode regime

extern "C" {

int cv3_linear_f32(const float* x, int64_t m, int64_t k, int64_t ldx, const float* w, int64_t ldw, int64_t n,
                   const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(m >= 0 && k > 0 && n >= 0 && ldw >= k && ldx >= k && ldy >= n, CV3_EINVAL,
              "bad linear shape m=%lld k=%lld n=%lld", (long long)m, (long long)k, (long long)n);
  if (!m || !n) return CV3_OK;
  hipStream_t st = stream_of(s);
  const bool rope = epi && epi->rope_cos;  // the rotary epilogue lives in the GEMM only
  if (m <= kGemvRows && !rope)
    return gemv(0, false, false, x, m, k, ldx, w, ldw * 4, nullptr, 1, k, n, bias, y, ldy, epi, nullptr, 0.f, st);
  return gemm(0, x, m, k, ldx, w, ldw, nullptr, false, 1, k, n, bias, y, ldy, epi, st);
}

int cv3_linear_q(int kind, const float* x, int64_t m, int64_t k, int64_t ldx, const void* q, const void* scales,
                 int scale_dtype, int64_t kp, int64_t block, int64_t n, const float* bias, float* y, int64_t ldy,
                 const cv3_epilogue* epi, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(kind == CV3_KIND_Q8 || kind == CV3_KIND_Q4, CV3_EINVAL, "unknown quant kind %d", kind);
  CV3_REQUIRE(m >= 0 && k > 0 && kp >= k && block > 0 && kp % block == 0 && ldx >= k && ldy >= n, CV3_EINVAL,
              "bad quantised linear shape m=%lld k=%lld kp=%lld block=%lld", (long long)m, (long long)k,
              (long long)kp, (long long)block);
  if (!m || !n) return CV3_OK;
  hipStream_t st = stream_of(s);
  const bool sf16 = scale_dtype == CV3_F16;
  const int64_t nb = kp / block;
  const bool rope = epi && epi->rope_cos;
  CV3_REQUIRE(!rope || kind == CV3_KIND_Q8, CV3_EUNSUPPORTED, "rotary epilogue on q4 weights");
  if (kind == CV3_KIND_Q8) {
    if (m <= kGemvRows && !rope)
      return gemv(1, sf16, false, x, m, k, ldx, q, kp, scales, nb, block, n, bias, y, ldy, epi, nullptr, 0.f, st);
    return gemm(1, x, m, k, ldx, q, kp, scales, sf16, nb, block, n, bias, y, ldy, epi, st);
  }
  // q4 (32-code blocks, float16 scales): the GEMV for the decode regime, the GEMM above it
  CV3_REQUIRE(block == 32, CV3_EUNSUPPORTED, "q4 weights need 32-code blocks (got %lld)", (long long)block);
  if (m <= kGemvRows)
    return gemv(2, true, false, x, m, k, ldx, q, kp / 2, scales, nb, block, n, bias, y, ldy, epi, nullptr, 0.f, st);
  return gemm(2, x, m, k, ldx, q, kp / 2, scales, true, nb, block, n, bias, y, ldy, epi, st);
}

// ops.linear with the weight held as three bfloat16 planes [3][n][ldp] (hi, mid, lo; the
// float32 weight to all 24 bits): the same float32 GEMM, on the bfloat16 matrix cores.
int cv3_split_x3(const float* w, int64_t n, int64_t k, int64_t ldw, uint16_t* planes, int64_t ldp, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(n >= 0 && k > 0 && ldw >= k && ldp >= k, CV3_EINVAL, "bad plane split shape n=%lld k=%lld",
              (long long)n, (long long)k);
  return split_x3(w, n, k, ldw, planes, ldp, n * ldp, stream_of(s));
}

int cv3_linear_x3(const float* x, int64_t m, int64_t k, int64_t ldx, const uint16_t* planes, int64_t ldp, int64_t n,
                  const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(m >= 0 && k > 0 && n >= 0 && ldp >= k && ldx >= k && ldy >= n, CV3_EINVAL,
              "bad linear shape m=%lld k=%lld n=%lld", (long long)m, (long long)k, (long long)n);
  if (!m || !n) return CV3_OK;
  return gemm_x3(x, m, k, ldx, planes, ldp, n * ldp, n, bias, y, ldy, epi, stream_of(s));
}

int cv3_split_x3_frag(const float* w, int64_t n, int64_t k, int64_t ldw, uint16_t* frag, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(n >= 0 && k > 0 && ldw >= k, CV3_EINVAL, "bad plane split shape n=%lld k=%lld", (long long)n,
              (long long)k);
  return split_x3_frag(w, n, k, ldw, frag, stream_of(s));
}

int cv3_x3_frag_elems(int64_t n, int64_t k, int64_t* elems) {
  CV3_REQUIRE(n >= 0 && k > 0 && elems, CV3_EINVAL, "bad shape or null output");
  *elems = 3 * x3_frag_plane(n, k);
  return CV3_OK;
}

int cv3_linear_x3_frag(const float* x, int64_t m, int64_t k, int64_t ldx, const uint16_t* frag, int64_t n,
                       const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(m >= 0 && k > 0 && n >= 0 && ldx >= k && ldy >= n, CV3_EINVAL, "bad linear shape m=%lld k=%lld n=%lld",
              (long long)m, (long long)k, (long long)n);
  if (!m || !n) return CV3_OK;
  return gemm_x3f(x, m, k, ldx, frag, n, bias, y, ldy, epi, stream_of(s));
}

int cv3_pack_q8_frag(const int8_t* q, int64_t n, int64_t k, int64_t ldq, int8_t* frag, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(n >= 0 && k > 0 && ldq >= k, CV3_EINVAL, "bad code pack shape n=%lld k=%lld", (long long)n,
              (long long)k);
  return pack_q8_frag(q, n, k, ldq, frag, stream_of(s));
}

int cv3_linear_q8_x3_frag(const float* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qfrag, const void* scales,
                          int scale_dtype, int64_t kp, int64_t block, int64_t n, const float* bias, float* y,
                          int64_t ldy, const cv3_epilogue* epi, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(m >= 0 && k > 0 && kp >= k && block > 0 && kp % block == 0 && ldx >= k && ldy >= n, CV3_EINVAL,
              "bad quantised linear shape m=%lld k=%lld kp=%lld block=%lld", (long long)m, (long long)k,
              (long long)kp, (long long)block);
  if (!m || !n) return CV3_OK;
  return gemm_x3qf(x, m, k, ldx, qfrag, scales, scale_dtype == CV3_F16, kp / block, block, n, bias, y, ldy, epi,
                   stream_of(s));
}

int cv3_pack_q8_frag32(const int8_t* q, int64_t n, int64_t k, int64_t ldq, int8_t* frag, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(n >= 0 && k > 0 && ldq >= k, CV3_EINVAL, "bad code pack shape n=%lld k=%lld", (long long)n,
              (long long)k);
  return pack_q8_frag32(q, n, k, ldq, frag, stream_of(s));
}

int cv3_linear_q8_digits(const float* x, int64_t m, int64_t k, int64_t ldx, const int8_t* qfrag32, const void* scales,
                         int scale_dtype, int64_t n, const float* bias, float* y, int64_t ldy, const cv3_epilogue* epi,
                         int32_t* row_exp, int row_exp_given, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(m >= 0 && k > 0 && ldx >= k && ldy >= n, CV3_EINVAL, "bad quantised linear shape m=%lld k=%lld",
              (long long)m, (long long)k);
  if (!m || !n) return CV3_OK;
  return gemm_q8d(x, m, k, ldx, qfrag32, scales, scale_dtype == CV3_F16, n, bias, y, ldy, epi, row_exp,
                  row_exp_given != 0, stream_of(s));
}

// quant.qmatmul on q8 weights (quant.py:165-190) with the activation as bfloat16 planes and
// the codes exact in bfloat16: three products per code, the block scale on each block sum.
int cv3_linear_q8_x3(const float* x, int64_t m, int64_t k, int64_t ldx, const int8_t* q, const void* scales,
                     int scale_dtype, int64_t kp, int64_t block, int64_t n, const float* bias, float* y, int64_t ldy,
                     const cv3_epilogue* epi, cv3_stream_t s) {
  CV3_ALIVE();
  CV3_REQUIRE(m >= 0 && k > 0 && kp >= k && block > 0 && kp % block == 0 && ldx >= k && ldy >= n, CV3_EINVAL,
              "bad quantised linear shape m=%lld k=%lld kp=%lld block=%lld", (long long)m, (long long)k,
              (long long)kp, (long long)block);
  if (!m || !n) return CV3_OK;
  return gemm_x3q(x, m, k, ldx, q, kp, scales, scale_dtype == CV3_F16, kp / block, block, n, bias, y, ldy, epi,
                  stream_of(s));
}

}  // extern "C"
