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

extern "C" int32_t kunserve_version(void) { return 300; }

extern "C" const char* kunserve_last_error(void) { return kunserve::g_last_error.c_str(); }

// ------------------------------------------------ fused page-id space
// A fusion group of N instances splits every base page of L layers into N
// pages of G = L / N layers (kunserve/block_manager.py:231-269). For a pool
// whose layers are contiguous within a page (page_stride == L *
// layer_stride, the [pages, layers, heads, slots, dim] layout), layer group
// i of page p is exactly page p * N + i of the same memory seen as
// [num_pages * N, G, heads, slots, dim]; the fused ids are a renumbering of
// those pages, so no kernel needs to know about fusion.

extern "C" int kunserve_fused_pool(const kunserve_kv_pool* pool, int64_t base_pages,
                                   int32_t fusion_size, kunserve_kv_pool* fused) {
  using namespace kunserve;
  clear_error();
  int rc = check_pool(pool, false);
  if (rc) return rc;
  KSV_CHECK_ARG(fused != nullptr, "null output pool");
  KSV_CHECK_ARG(fusion_size >= 1 && pool->num_layers % fusion_size == 0,
                "%d layers do not split into %d equal stages", pool->num_layers, fusion_size);
  KSV_CHECK_ARG(base_pages >= 1 && base_pages <= pool->num_pages,
                "base_pages %lld outside [1, %lld]", (long long)base_pages,
                (long long)pool->num_pages);
  if (pool->page_stride != int64_t(pool->num_layers) * pool->layer_stride) {
    set_error("fused pages need the layers of a page to be contiguous (page_stride %lld != "
              "%d layers x layer_stride %lld)", (long long)pool->page_stride, pool->num_layers,
              (long long)pool->layer_stride);
    return KUNSERVE_EUNSUPPORTED;
  }
  const int64_t pages = pool->num_pages * fusion_size;
  KSV_CHECK_ARG(pages < (int64_t(1) << 31), "%lld fused pages exceed 2^31", (long long)pages);
  *fused = *pool;
  fused->num_pages = pages;
  fused->num_layers = pool->num_layers / fusion_size;
  fused->page_stride = int64_t(fused->num_layers) * pool->layer_stride;
  return KUNSERVE_OK;
}

extern "C" int kunserve_fused_page_ids(const int32_t* fused_ids_host, int64_t n,
                                       int64_t base_pages, int32_t fusion_size,
                                       int64_t num_fused_pages, int32_t* pages_host) {
  using namespace kunserve;
  clear_error();
  KSV_CHECK_ARG(n >= 0 && (n == 0 || (fused_ids_host && pages_host)), "null id array");
  KSV_CHECK_ARG(fusion_size >= 1 && base_pages >= 1, "bad fusion geometry");
  const int64_t base_ids = base_pages * fusion_size;
  KSV_CHECK_ARG(num_fused_pages >= base_ids && num_fused_pages < (int64_t(1) << 31),
                "num_fused_pages %lld below the %lld fused base pages",
                (long long)num_fused_pages, (long long)base_ids);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t f = fused_ids_host[i];
    if (f < 0 || f >= num_fused_pages) {
      set_error("fused page id %lld outside [0, %lld)", (long long)f, (long long)num_fused_pages);
      return KUNSERVE_ERANGE;
    }
    // Base ids i * P + b -> page b * N + i; extend ids (>= P * N) map to
    // themselves: extend page P + q of the unfused pool is fused pages
    // (P + q) * N + i = P * N + (q * N + i).
    pages_host[i] = f < base_ids ? int32_t((f % base_pages) * fusion_size + f / base_pages)
                                 : int32_t(f);
  }
  return KUNSERVE_OK;
}
