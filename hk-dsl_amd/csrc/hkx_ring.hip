// The persistent ring GEMM kernel (hkx_ring.hpp): which instantiation a call takes.
#include "hkx_launch.hpp"
#include "hkx_ring.hpp"

namespace hkx {

namespace {

bool vec16(const Opnd& o) { return o.p && o.ld != 0 && o.dt == HKX_BF16; }
bool vec32(const Opnd& o) { return o.p && o.ld != 0 && o.dt == HKX_FP32; }

// The compiled epilogue form for a fused epilogue (kEpGeneric when no faster form fits).
int ring_form(const TileArgs& a, bool fp8, int mode) {
  const Fused& e = a.ep;
  if (mode != kStore16) return kEpGeneric;
  if (e.form != HKX_EP_FUSED) return kEpNone;
  if (a.c_dt != HKX_BF16 || e.ta.p || e.cmul != 1.0f || e.cadd != 0.0f) return kEpGeneric;
  if (!e.cs.p && !e.rs.p && !e.ra.p) return kEpNone;
  if (!e.cs.p && !e.rs.p && vec16(e.ra)) return kEpBias;
  if (fp8 && vec32(e.cs) && vec32(e.rs) && e.act == HKX_ACT_NONE) {
    if (!e.ra.p) return kEpDeq;
    if (vec16(e.ra)) return kEpDeqBias;
  }
  return kEpGeneric;
}

}  // namespace

bool ring_takes(const TileArgs& a, bool fp8, int mode) {
  const int ob = mode == kStore8 ? 1 : (mode == kStoreF32 || mode == kPairWs ? 4 : 2);
  if (fp8 && (mode == kPair16 || mode == kPairWs)) return false;
  // whole 16-byte (8-byte for 8-bit C) pieces of rows
  if (ob != 4 && (a.N % 8 || !a.c_aligned || (a.ldc * ob) % 16)) return false;
  // C (one split's share) is stored through a buffer resource with 32-bit byte offsets,
  // computed for every row of the last (ragged) 256-row tile, the rows past M included:
  // those rows' offsets must not wrap round into C's first rows.
  if ((int64_t)((a.M + 255) / 256) * 256 * a.ldc * ob >= (1LL << 32)) return false;
  // a 16-bit column scale is read as aligned pairs: unit stride only
  const Opnd& cs = a.ep.cs;
  if (a.ep.form == HKX_EP_FUSED && cs.p && cs.ld && cs.dt != HKX_FP32 && cs.ld != 1) return false;
  // and from a 4-byte aligned address (the slot of an element is the aligned word it starts)
  if (a.ep.form == HKX_EP_FUSED)
    for (const Opnd* o : {&a.ep.cs, &a.ep.rs, &a.ep.ra})
      if (o->p && o->ld && o->dt != HKX_FP32 && ((uintptr_t)o->p & 3)) return false;
  return true;
}

hipError_t launch_ring(const TileArgs& a, bool fp8, int mode, dim3 grid, hipStream_t s) {
  if (!ring_takes(a, fp8, mode)) return hipErrorInvalidValue;
  const int epf = ring_form(a, fp8, mode);
  const int act = a.ep.form == HKX_EP_FUSED ? a.ep.act : HKX_ACT_NONE;
  return fp8 ? launch_ring_fp8(a, mode, epf, act, grid, s)
             : launch_ring_bf16(a, mode, epf, act, grid, s);
}

}  // namespace hkx
