/* kt_launch.h - every launch of the library goes through kt_go: it launches the kernel on the stream, or, while the
   calling thread is recording (kt_record_begin .. kt_record_end, include/kt.h), appends a launch record instead:
   the kernel's hipFunction_t (hipGetFuncBySymbol), grid, block, dynamic LDS bytes and the argument values converted
   to the kernel's parameter types, with the kernelParams array hipModuleLaunchKernel takes. That is the tuple Kindi's
   plan holds for each launch (Plan.add, tp.py:282-302) and replays (Replay.launch, spec.py:303-320). */
#pragma once
#include <hip/hip_runtime.h>
#include <cstring>
#include <tuple>
#include <type_traits>
#include <utility>
#include "../../include/kt.h"

struct KtRecState {
  kt_launch* buf;
  int max, n;                          /* capacity; launches seen (n > max: overflow, reported by kt_record_end) */
  int err;                             /* the first error while recording */
};
KtRecState* kt_rec_state();            /* the calling thread's recording, or nullptr */

/* one record: the values vals[i] (sizes[i] bytes, aligned to aligns[i]) in the record's own argument buffer */
hipError_t kt_rec_push(const void* fn, dim3 g, dim3 b, size_t lds, int n, const void* const* vals,
                       const size_t* sizes, const size_t* aligns);

template <typename Tup, size_t... I>
static inline hipError_t kt_rec_tuple(const void* fn, dim3 g, dim3 b, size_t lds, const Tup& t,
                                      std::index_sequence<I...>){
  constexpr int n = (int)sizeof...(I);
  const void* vals[n > 0 ? n : 1] = {(const void*)&std::get<I>(t)...};
  const size_t sizes[n > 0 ? n : 1] = {sizeof(std::tuple_element_t<I, Tup>)...};
  const size_t aligns[n > 0 ? n : 1] = {alignof(std::tuple_element_t<I, Tup>)...};
  return kt_rec_push(fn, g, b, lds, n, vals, sizes, aligns);
}

template <typename... P, typename... A>
static inline hipError_t kt_go(void (*k)(P...), dim3 g, dim3 b, size_t lds, hipStream_t s, A... a){
  static_assert(sizeof...(P) == sizeof...(A), "kt_go: argument count");
  if(KtRecState* r = kt_rec_state()){
    /* the values as the kernel's parameter types (the conversions a launch makes) */
    const std::tuple<std::remove_cv_t<std::remove_reference_t<P>>...> t(a...);
    return kt_rec_tuple((const void*)k, g, b, lds, t, std::index_sequence_for<P...>{});
  }
  hipLaunchKernelGGL(k, g, b, lds, s, a...);
  return hipGetLastError();
}

/* launch (or record) and return the error from the calling entry point */
#define KT_LAUNCH(K, G, B, LDS, S, ...) do { const hipError_t _le = kt_go((K), (G), (B), (LDS), (S), __VA_ARGS__); \
    if(_le != hipSuccess) return (int)_le; } while(0)
