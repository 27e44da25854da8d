// The merge and cache-write items that follow the decode kernel, shared by
// the finish kernel (rpa_finish.hip) and the finish workgroups of the prefill
// kernel (rpa_prefill.hip).  Both launch after the decode kernel on the same
// stream, so its partials and published plan are visible to plain loads.
//
//   merge  item it < n * Hkv: pair (s, h) = (it / Hkv, it % Hkv) of a decode
//          sequence cut between several decode wavefronts (rpa_plan.h):
//          combine the partials in slots w_a + it .. w_b + it (rpa_merge.h).
//   write  token row t of a non-decode sequence: its new K/V record into its
//          cache page (kernel.py:154-166), unless skip_kv_update.
#pragma once

#include "rpa_common.h"
#include "rpa_generic_row.h"
#include "rpa_internal.h"
#include "rpa_merge.h"
#include "rpa_plan.h"

namespace rpa {

// Merge item `it` (pair index, it < S * Hkv) with the decode kernel's
// published plan.  The plan header (sequence count n, tiles per wavefront)
// and the item's entries are loaded together -- one memory round trip before
// the partials' -- and an empty asm that reads them all keeps the compiler
// from sinking any of them below the tests.  Entries of sequences past n are
// stale but inside the plan, and are discarded.  Returns false when the
// item's sequence is past n (so is every later item's).
template <int DP, typename OutS>
__device__ __forceinline__ bool finish_merge_item(const Params& p, const PlanView& pv, int32_t it,
                                                  const int32_t* __restrict__ cu,
                                                  const float* __restrict__ part_o,
                                                  const float* __restrict__ part_ml,
                                                  OutS* __restrict__ out) {
  const int32_t s = it / p.Hkv;
  const int32_t h = it - s * p.Hkv;
  // (The header is indexed by a zero that an asm produces, so that its loads
  // are not hoisted out of the caller's loop -- and waited on -- ahead of
  // the item's loads.)
  int32_t z = 0;
  asm volatile("" : "+v"(z));
  int32_t hn = pv.hdr[z], htpw = pv.hdr[z + 1];
  int32_t b0 = pv.base[s], b1 = pv.base[s + 1], dkv = pv.dkv[s], tq = pv.tq[s];
  int32_t c0 = cu[s], c1 = cu[s + 1];
  asm volatile("" : "+v"(hn), "+v"(htpw), "+v"(b0), "+v"(b1), "+v"(dkv), "+v"(tq), "+v"(c0),
               "+v"(c1));
  const int32_t n = min(max(hn, 0), p.S);
  const int32_t tpw = max(htpw, 1);
  // The pair's tiles [g0, g0 + nt) of the work line; the wavefronts owning
  // its first and last tile, and its partial slots w + pair.
  const int32_t nt = b1 - b0;
  if (s >= n) return false;
  if (dkv == 0 || nt <= 0) return true;
  const int32_t g0 = p.Hkv * b0 + h * nt;
  const int32_t wa = g0 / tpw, wb = (g0 + nt - 1) / tpw;
  if (wa == wb) return true;  // one wavefront finished the pair
  const int32_t first = wa + it;
  const int32_t nparts = wb - wa + 1;
  // The decode group's rows: q_len tokens x qpk heads (q_len * qpk <= 16).
  const int32_t ql = p.dq > 1 ? min(max(c1 - c0, 1), p.dq) : 1;
  const int32_t rows = min(ql * p.qpk, 16);
  switch (decode_slot_rows(p.qpk * p.dq)) {
    case 1: merge_partials<DP, 1>(p, part_o, part_ml, first, nparts, rows, out, tq, h); break;
    case 2: merge_partials<DP, 2>(p, part_o, part_ml, first, nparts, rows, out, tq, h); break;
    case 4: merge_partials<DP, 4>(p, part_o, part_ml, first, nparts, rows, out, tq, h); break;
    case 8: merge_partials<DP, 8>(p, part_o, part_ml, first, nparts, rows, out, tq, h); break;
    default: merge_partials<DP, 16>(p, part_o, part_ml, first, nparts, rows, out, tq, h); break;
  }
  return true;
}

// Sequence that owns token row t for the row items: with the decode kernel's
// plan (rowseq: -1 for decode and padding rows), else from the plan rows R
// that this workgroup built in LDS.  Returns false when no sequence's
// non-decode rows contain t.
struct RowOwner {
  int32_t s, q_start, q_end, kv_len;
};
__device__ __forceinline__ bool row_owner(const Params& p, bool decode_on, const PlanView& pv,
                                          const PlanRows* R, int32_t n, const int32_t* cu,
                                          const int32_t* kv_lens, int32_t t, RowOwner* o) {
  if (decode_on) {
    o->s = pv.rowseq[t];
    if (o->s < 0 || o->s >= n) return false;
    o->q_start = cu[o->s];
    o->q_end = cu[o->s + 1];
    o->kv_len = min(kv_lens[o->s], p.pps * p.ps);
  } else {
    o->s = find_seq(R->cu, n + 1, t);
    if (o->s < 0 || o->s >= n) return false;
    o->q_start = R->cu[o->s];
    o->q_end = R->cu[o->s + 1];
    o->kv_len = R->kvlen[o->s];
  }
  return t >= o->q_start && t < o->q_end;
}

// Write item for token row t.
template <typename E>
__device__ __forceinline__ void finish_write_item(const Params& p, bool decode_on,
                                                  const PlanView& pv, const PlanRows* R,
                                                  int32_t n, const int32_t* cu,
                                                  const int32_t* kv_lens, E* __restrict__ cache,
                                                  const int32_t* __restrict__ page_indices,
                                                  const E* __restrict__ keys,
                                                  const E* __restrict__ values, int32_t t,
                                                  int lane) {
  RowOwner o;
  if (!row_owner(p, decode_on, pv, R, n, cu, kv_lens, t, &o)) return;
  const int32_t j = o.kv_len - (o.q_end - o.q_start) + (t - o.q_start);
  if (j >= 0) write_record<E>(p, cache, page_indices, keys, values, o.s, j, t, lane);
}

}  // namespace rpa
