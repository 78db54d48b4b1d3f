// The attention output block as one persistent gfx950 launch: the merged latent o_lat
// through W_UV per head, then o_proj and the residual add of the W == 1 reduce.
//   1  W_UV: o[r][h * 128 + v] = sum_c W_UV[h][v][c] o_lat[r][h][c] (32 groups of
//      [128, 512], two 16-row groups a task), handed over in bf16 (the reference rounds
//      o to bf16 before W_UV's output goes on, kernel.py:4080-4123).
//   2  o_proj: a[r][n] = bf16(h[r][n] + sum_k W_o[n][k] o[r][k]) ([7168, 4096], one 16-row
//      group a task, 16 K-splits). Its first weights are in flight before the wait for
//      every CTA's W_UV outputs.
// Reference: sgl_amd_mono/glm53/gfx950/kernel.py:3975-4123 (W_UV), :4125-4197 (o_proj,
// residual), :1665-1669 (W == 1 reduce).
#include <hip/hip_runtime.h>

#include "gemv.h"
#include "mono_abi.h"

namespace mono {

constexpr int PO_HEADS = 32, PO_V = 128, PO_LAT = 512, PO_HID = 7168;
constexpr int PO_O = PO_HEADS * PO_V;
constexpr int PO_MAXR = 16;
constexpr int PO_MAX_GRID = 1024;

struct PostScratch {
  static constexpr size_t O = 0;  // bf16 [16][4096]
  static constexpr size_t DONE = (O + (size_t)PO_MAXR * PO_O * 2 + 255) & ~(size_t)255;
  static constexpr size_t BYTES = (DONE + PO_MAX_GRID * 4 + 255) & ~(size_t)255;
};

struct PostParams {
  int rows, shuf;
  const uint16_t* o_lat;
  const uint16_t* h;
  const uint8_t* w_uv;
  const float* s_uv;
  const uint8_t* w_o;
  const float* s_o;
  uint16_t* out;
  uint16_t* o;  // bf16 [R][4096]: the caller's, or scratch
  uint8_t* scratch;
  int32_t* guard;
  uint32_t* host_err;
  int fault_site, fault_after;
  uint64_t* timeline;
};

__global__ void __launch_bounds__(1024, 1) post_kernel(PostParams p) {
  const int b = blockIdx.x, nblk = gridDim.x, R = p.rows;
  __shared__ v4f red[16][64];
  __shared__ uint32_t head_s[4];
  __shared__ int ok_s;
  uint32_t* done = reinterpret_cast<uint32_t*>(p.scratch + PostScratch::DONE);

  stamp(p.timeline, MONO_TL_START);
  if (threadIdx.x == 0) {
    const v4i hd = ld16<CP_DEV>(rsrc(p.guard, 16), 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) head_s[i] = (uint32_t)hd[i];
    ok_s = 1;
  }
  __syncthreads();
  const uint32_t tag = head_s[MONO_GUARD_EPOCH] + 1u;
  Guard guard;
  guard.init(p.guard, p.host_err, p.fault_site, head_s, (uint32_t)p.fault_after);

  // ---------------------------------------------------------------- 1: W_UV
  {
    const int tid = opaque_v((int)threadIdx.x);
    GemvJob j{};
    j.x = p.o_lat;
    j.x_stride = PO_HEADS * PO_LAT;
    j.x_gstride = PO_LAT;
    j.w = p.w_uv;
    j.s = p.s_uv;
    j.N = PO_V;
    j.K = PO_LAT;
    j.G = PO_HEADS;
    j.shuf = p.shuf;
    j.out_bf = p.o;
    j.out_stride = PO_O;
    j.out_gstride = PO_V;
    gemv_tasks<8, 1, CP_NONE>(j, R, b, nblk, tid, red, []() { return true; });
    // the epilogue threads (waves 0-7) made every store: once they completed, the CTA's
    // done word takes the launch tag
    if (tid < 512) drain();
    __syncthreads();
    if (tid == 0) st_dev(&done[b], tag);
  }

  // ---------------------------------------------------------------- 2: o_proj
  stamp(p.timeline, MONO_TL_STAGED);
  bool ok = true;
  {
    const int tid = opaque_v((int)threadIdx.x);
    const int l = tid & 63, w = tid >> 6;
    GemvJob j{};
    j.x = p.o;
    j.x_stride = PO_O;
    j.x_gstride = 0;
    j.w = p.w_o;
    j.s = p.s_o;
    j.N = PO_HID;
    j.K = PO_O;
    j.G = 1;
    j.shuf = p.shuf;
    j.out_bf = p.out;
    j.out_stride = PO_HID;
    j.res = p.h;
    j.res_stride = PO_HID;
    ok = gemv_tasks<16, 4, CP_DEV>(j, R, b, nblk, tid, red, [&]() {
      bool got = true;
      if (w == 15)  // one wave polls; the CTA's first weights stay in flight meanwhile
        got = wait_until(guard, MONO_SITE_O, [&]() {
          bool all = true;
          for (int i = l; i < nblk; i += WAVE) all &= ld_dev(&done[i]) == tag;
          return __all(all);
        });
      return cta_all(got, ok_s);
    });
  }
  (void)ok;

  // ---------------------------------------------------------------- exit
  stamp(p.timeline, MONO_TL_ROUTED);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* gw = reinterpret_cast<uint32_t*>(p.guard);
    drain();
    const uint32_t old = add_dev(gw + MONO_GUARD_EXIT, 1u);
    if (old == (uint32_t)nblk - 1u) {
      st_dev(gw + MONO_GUARD_EXIT, 0u);
      st_dev(gw + MONO_GUARD_EPOCH, tag);
    }
  }
  stamp(p.timeline, MONO_TL_END);
}

}  // namespace mono

using namespace mono;

extern "C" size_t mono_post_scratch_bytes(void) { return PostScratch::BYTES; }

extern "C" int mono_post_launch(const MonoPostArgs* a, mono_stream_t stream) {
  if (!a) return set_error(MONO_E_ARG, "mono_post_launch: null args");
  if (a->rows < 1 || a->rows > PO_MAXR)
    return set_error(MONO_E_ARG, "mono_post_launch: rows must be 1..16");
  if (a->heads != PO_HEADS || a->hidden != PO_HID)
    return set_error(MONO_E_ARG, "mono_post_launch: built for 32 heads and hidden 7168");
  if (a->layout != MONO_LAYOUT_ROWMAJOR && a->layout != MONO_LAYOUT_AITER16)
    return set_error(MONO_E_ARG, "mono_post_launch: unknown weight layout");
  if (!a->o_lat || !a->h || !a->w_uv || !a->s_uv || !a->w_o || !a->s_o || !a->out ||
      !a->scratch || !a->guard)
    return set_error(MONO_E_ARG, "mono_post_launch: null tensor");
  PostParams p;
  p.rows = a->rows;
  p.shuf = a->layout == MONO_LAYOUT_AITER16;
  p.o_lat = static_cast<const uint16_t*>(a->o_lat);
  p.h = static_cast<const uint16_t*>(a->h);
  p.w_uv = a->w_uv;
  p.s_uv = a->s_uv;
  p.w_o = a->w_o;
  p.s_o = a->s_o;
  p.out = static_cast<uint16_t*>(a->out);
  p.scratch = static_cast<uint8_t*>(a->scratch);
  p.o = a->o ? static_cast<uint16_t*>(a->o)
             : reinterpret_cast<uint16_t*>(p.scratch + PostScratch::O);
  p.guard = a->guard;
  p.host_err = nullptr;
  if (a->host_error) {
    void* dptr = nullptr;
    if (hipHostGetDevicePointer(&dptr, a->host_error, 0) != hipSuccess || !dptr)
      return set_error(MONO_E_ARG, "mono_post_launch: host_error is not pinned host memory");
    p.host_err = static_cast<uint32_t*>(dptr);
  }
  p.fault_site = a->fault_site;
  p.fault_after = a->fault_after;
  p.timeline = a->timeline;
  int grid = 0;
  int rc = monokernel_grid(&grid);
  if (rc) return rc;
  if (grid > PO_MAX_GRID) return set_error(MONO_E_DEVICE, "mono_post_launch: grid too large");
  rc = check_coresident(post_kernel, 1024, 0,
                        "mono_post_launch: one 1024-thread CTA per CU does not fit");
  if (rc) return rc;
  hipLaunchKernelGGL(post_kernel, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
  return check_launch("mono_post_launch");
}
