// hv_image.hip -- image front end: float CHW images quantised to int8 at the
// input exponent (p2_export_weights.real_image_list, tools/p2/
// p2_export_weights.py:246-251; p2_sim.forward_image, tools/p2/p2_sim.py:
// 536-543), written either as the flat NHWC image the golden model takes or
// directly as the patch matrix of the patch embedding (layout.patchify,
// layout.py:31-72), so the patch GEMM reads contiguous 768-byte rows.
#include "hv_device.h"
#include "hv_internal.h"

namespace hv {

// q = clamp(round_half_even(x / 2^exp), -128, 127).  x * 2^-exp is the same
// correctly rounded float32 as the division (a power of two, |exp| <= 32);
// NaN, whose int8 cast the reference leaves undefined, maps to 0.
__device__ __forceinline__ int quant_px(float x, float scale) {
  const float v = rintf(x * scale);
  if (v != v) return 0;
  return (int)fminf(fmaxf(v, -128.f), 127.f);
}

// One work item: 4 horizontally adjacent pixels of one image row, all three
// channels (three coalesced 16-byte loads, one per channel plane); they are
// 12 contiguous output bytes in both layouts.  Items stride over the batch.
template <bool PATCH_ROWS>
__global__ __launch_bounds__(256) void k_image_front(const float *__restrict__ chw, int batch,
                                                     float scale, int8_t *__restrict__ out) {
  constexpr int kQuads = 56, kRows = 224, kPlane = 224 * 224;
  const long long items = (long long)batch * kRows * kQuads;
  for (long long i = blockIdx.x * 256ll + threadIdx.x; i < items; i += gridDim.x * 256ll) {
    const int b = (int)(i / (kRows * kQuads));
    const int rem = (int)(i - (long long)b * kRows * kQuads);
    const int y = rem / kQuads, x0 = (rem - y * kQuads) * 4;
    const float *src = chw + (size_t)b * 3 * kPlane + y * 224 + x0;
    const float4 c0 = *reinterpret_cast<const float4 *>(src);
    const float4 c1 = *reinterpret_cast<const float4 *>(src + kPlane);
    const float4 c2 = *reinterpret_cast<const float4 *>(src + 2 * kPlane);
    const int q[12] = {quant_px(c0.x, scale), quant_px(c1.x, scale), quant_px(c2.x, scale),
                       quant_px(c0.y, scale), quant_px(c1.y, scale), quant_px(c2.y, scale),
                       quant_px(c0.z, scale), quant_px(c1.z, scale), quant_px(c2.z, scale),
                       quant_px(c0.w, scale), quant_px(c1.w, scale), quant_px(c2.w, scale)};
    int w[3];
#pragma unroll
    for (int j = 0; j < 3; ++j)
      w[j] = (q[4 * j] & 0xFF) | (q[4 * j + 1] & 0xFF) << 8 | (q[4 * j + 2] & 0xFF) << 16 |
             (q[4 * j + 3] & 0xFF) << 24;
    size_t off;
    if (PATCH_ROWS) {
      // patch pr*14 + pc, column (in_row*16 + in_col)*3 + ch
      const int pr = y >> 4, in_row = y & 15, pc = x0 >> 4, in_col = x0 & 15;
      off = ((size_t)b * 196 + pr * 14 + pc) * 768 + in_row * 48 + in_col * 3;
    } else {
      off = (((size_t)b * 224 + y) * 224 + x0) * 3;
    }
    int *dst = reinterpret_cast<int *>(out + off);
    dst[0] = w[0];
    dst[1] = w[1];
    dst[2] = w[2];
  }
}

int launch_image_front(const float *chw, int batch, int input_exp, int8_t *out, bool patch_rows,
                       hipStream_t s) {
  if (input_exp < -32 || input_exp > 31)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "input scale exponent %d outside [-32, 31]",
                input_exp);
  if (((uintptr_t)chw & 15) || ((uintptr_t)out & 3))
    return fail(HV_EVALUE, HV_ERR_ADDRESS,
                "images: float input must be 16-byte and output 4-byte aligned");
  if (batch <= 0) return HV_OK;
  const float scale = ldexpf(1.f, -input_exp);
  const long long items = (long long)batch * 224 * 56;
  const long long blocks = (items + 255) / 256;
  const dim3 grid((unsigned)(blocks < 256 * 8 ? blocks : 256 * 8)), block(256);
  if (patch_rows) hv_launch(k_image_front<true>, grid, block, 0, s, chw, batch, scale, out);
  else hv_launch(k_image_front<false>, grid, block, 0, s, chw, batch, scale, out);
  return check_hip(hipGetLastError(), "k_image_front launch");
}

}  // namespace hv
