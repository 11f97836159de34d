// Host-side helpers shared by the C-ABI entry points: thread-local error
// message, argument checks, launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "dimmerkv.h"

namespace dkv {

void set_error(const char* fmt, ...);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return DKV_ELAUNCH;
  }
  return DKV_OK;
}

inline int check_order(const dkv_order_t& o, const char* what) {
  if (o.groups <= 0 || o.pieces <= 0 || o.pieces > 8 * o.groups) {
    set_error("%s: bad order (groups=%d pieces=%d)", what, o.groups, o.pieces);
    return DKV_ESHAPE;
  }
  if (!o.planes || !o.seg_off || !o.prefix_bytes) {
    set_error("%s: order tables must be non-null", what);
    return DKV_EINVAL;
  }
  return DKV_OK;
}

inline int check_ladder(const dkv_ladder_t& l, const char* what) {
  if (l.groups <= 0 || l.rungs <= 0) {
    set_error("%s: bad ladder (groups=%d rungs=%d)", what, l.groups, l.rungs);
    return DKV_ESHAPE;
  }
  if (!l.bits || !l.seg_off || !l.rung_bytes) {
    set_error("%s: ladder tables must be non-null", what);
    return DKV_EINVAL;
  }
  return DKV_OK;
}

inline int check_stream(const dkv_stream_t* s, const char* what) {
  if (!s || !s->blob || !s->tok_off || !s->pieces) {
    set_error("%s: stream blob/tok_off/pieces must be non-null", what);
    return DKV_EINVAL;
  }
  if (s->format == DKV_FMT_LADDER) return check_ladder(s->ladder, what);
  if (s->format != DKV_FMT_PLANES) {
    set_error("%s: unknown stream format %d", what, s->format);
    return DKV_EINVAL;
  }
  return check_order(s->order, what);
}

// 64-component groups of a (checked) stream.
inline int stream_groups(const dkv_stream_t& s) {
  return s.format == DKV_FMT_LADDER ? s.ladder.groups : s.order.groups;
}

}  // namespace dkv

#define DKV_REQUIRE(cond, code, ...)   \
  do {                                 \
    if (!(cond)) {                     \
      dkv::set_error(__VA_ARGS__);     \
      return (code);                   \
    }                                  \
  } while (0)
