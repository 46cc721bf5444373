// npa_sort.hip - stable radix sort of indices by 32-bit keys (rocPRIM's device radix sort), used
// for the oriented raster's depth order. LSD radix sorting is stable: equal keys keep ascending
// index order.
#include <hip/hip_runtime.h>

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/iterator/counting_iterator.hpp>

#include "npa_internal.hpp"

namespace npa {

hipError_t sort_index_by_key(const uint32_t* keys, uint32_t* keys_out, uint32_t* order, uint32_t n,
                             uint32_t end_bit, DevBuf& temp, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const auto idx = rocprim::make_counting_iterator<uint32_t>(0u);
    size_t bytes = 0;
    hipError_t e = rocprim::radix_sort_pairs(nullptr, bytes, keys, keys_out, idx, order, n, 0u, end_bit, stream);
    if (e != hipSuccess) return e;
    if ((e = temp.reserve(bytes ? bytes : 1)) != hipSuccess) return e;
    return rocprim::radix_sort_pairs(temp.ptr, bytes, keys, keys_out, idx, order, n, 0u, end_bit, stream);
}

}  // namespace npa
