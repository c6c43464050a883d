// Weight-template rebasing shared by the .animapk reader and the streamed DiT forward:
// a template's buffer pointer holds a byte offset from the start of its execution range
// (DiTQuantizedWeightFactory.makeMatrix binds ring + tensor offset the same way,
// AnimaXS/Runtime/Metal/LinearExecutor.swift:467-518).  Host-only.
#pragma once

#include "anima_hip.h"

namespace anima {

// {base + offset, range_bytes - offset}; ANIMA_E_OUT_OF_BOUNDS when the offset lies past
// the range.
anima_buffer rebase_buffer(const anima_buffer& t, char* base, int64_t range_bytes, const char* what);
anima_qweight rebase_qweight(const anima_qweight& t, char* base, int64_t range_bytes, const char* what);
anima_dit_block_weights rebase_block(const anima_dit_block_weights& t, char* base, int64_t range_bytes);

}  // namespace anima
