// Error reporting and argument checks shared by the C ABI entry points.
#include "common.hpp"

namespace kunserve {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_pool(const kunserve_kv_pool* p, bool need_vec_align) {
  KSV_CHECK_ARG(p != nullptr, "null pool");
  KSV_CHECK_ARG(p->k && p->v, "null K or V pool pointer");
  KSV_CHECK_ARG(p->num_pages > 0 && p->num_pages < (int64_t(1) << 31),
                "num_pages %lld outside [1, 2^31)", (long long)p->num_pages);
  KSV_CHECK_ARG(p->num_layers > 0 && p->num_kv_heads > 0, "empty pool geometry");
  KSV_CHECK_ARG(p->page_size >= 4 && (p->page_size & (p->page_size - 1)) == 0,
                "page_size %d must be a power of two >= 4", p->page_size);
  KSV_CHECK_ARG(p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256,
                "head_dim %d not in {64, 128, 256}", p->head_dim);
  KSV_CHECK_ARG(p->dtype == KUNSERVE_DTYPE_F16 || p->dtype == KUNSERVE_DTYPE_BF16,
                "dtype %d is neither KUNSERVE_DTYPE_F16 nor KUNSERVE_DTYPE_BF16", p->dtype);
  KSV_CHECK_ARG(p->page_stride > 0 && p->layer_stride >= 0 && p->head_stride >= 0 &&
                    p->token_stride >= p->head_dim,
                "bad pool strides");
  if (need_vec_align) {
    KSV_CHECK_ARG(aligned16(p->k) && aligned16(p->v), "pool base must be 16-byte aligned");
    KSV_CHECK_ARG(p->page_stride % 8 == 0 && p->layer_stride % 8 == 0 &&
                      p->head_stride % 8 == 0 && p->token_stride % 8 == 0,
                  "pool strides must be multiples of 8 elements");
  } else {
    KSV_CHECK_ARG(aligned16(p->k) && aligned16(p->v) && p->page_stride % 8 == 0 &&
                      p->layer_stride % 8 == 0,
                  "pool base and page/layer strides must be 16-byte aligned");
  }
  return KUNSERVE_OK;
}

}  // namespace kunserve

extern "C" int32_t kunserve_version(void) { return 100; }

extern "C" const char* kunserve_last_error(void) { return kunserve::g_last_error.c_str(); }
