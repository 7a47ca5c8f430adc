/* Compile-time check that the mirrors in include/ibhip.h are layout-identical
 * to the reference's structs: ibh_kernels vs ib_kernels
 * (src/inferbit_internal.h:199-277), ibh_ref_pq_tensor vs ib_pq_tensor
 * (src/pq_decode.h:39-87).  Built by tests/test_layout.py against the
 * reference headers; it only has to compile. */
#include <stddef.h>

#include "ibhip.h"
#include "inferbit_internal.h"
#include "pq_decode.h"

#define SAME(A, B, f) _Static_assert(offsetof(A, f) == offsetof(B, f), #A "." #f " offset");

_Static_assert(sizeof(ibh_kernels) == sizeof(ib_kernels), "ibh_kernels size");
SAME(ibh_kernels, ib_kernels, matmul_int4)
SAME(ibh_kernels, ib_kernels, matmul_int8)
SAME(ibh_kernels, ib_kernels, matmul_int2)
SAME(ibh_kernels, ib_kernels, rmsnorm)
SAME(ibh_kernels, ib_kernels, rope)
SAME(ibh_kernels, ib_kernels, softmax)
SAME(ibh_kernels, ib_kernels, silu_mul)
SAME(ibh_kernels, ib_kernels, matmul_w4a8)
SAME(ibh_kernels, ib_kernels, matmul_w4a8_batch)
SAME(ibh_kernels, ib_kernels, matmul_int8_batch)

_Static_assert(sizeof(ibh_ref_pq_tensor) == sizeof(ib_pq_tensor), "ibh_ref_pq_tensor size");
_Static_assert(sizeof(((ib_pq_tensor*)0)->format) == sizeof(int), "ib_pq_format is an int");
SAME(ibh_ref_pq_tensor, ib_pq_tensor, M)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, N)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, G)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, K)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, K_l2)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, n_levels)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, rotate)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, n_outlier)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, format)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, codebook_l1_l)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, codebook_l1_r)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, codebook_l2_l)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, codebook_l2_r)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, indices_l1_l)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, indices_l1_r)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, indices_l2_l)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, indices_l2_r)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, C)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, l2_idx_bytes)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, l2_packed_bits)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, row_scale)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, outlier_cols)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, outlier_sidecar)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, outlier_scale)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, _arena)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, _arena_size)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, _mmap_base)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, _mmap_size)
SAME(ibh_ref_pq_tensor, ib_pq_tensor, _owns_mmap)

/* the host twin takes the reference's struct pointer as it is */
static int (*const twin)(const ibh_ref_pq_tensor*, const float*, float*) = ibh_pq_matmul_fp32_host;
int layout_check_use(const ib_pq_tensor* t, const float* x, float* y) { return twin((const ibh_ref_pq_tensor*)t, x, y); }
