// fbgemm_cpu.cpp -- TEST INFRASTRUCTURE ONLY.  A thin C harness over FBGEMM's
// CPU embedding kernels as exported by the installed torch
// (libtorch_cpu.so; declarations in torch/include/fbgemm/FbgemmEmbedding.h).
// These are the CPU kernels fbgemm_gpu's CPU TBE operators wrap, so they
// serve two roles here: an independent pin for the C restatement in
// mx_oracle.c, and the CPU baseline that bench.py times on the GPU box's
// host cores.  Nothing in the product links or loads this file.
//
// Layout notes (FbgemmEmbedding.h): output_stride / input_stride let one
// kernel call write a table's D-slice of the [B, total_D] output and read
// padded rows; scale_bias_last = false selects the TBE row layout (fp16
// scale and bias at the front of each quantized row, :88-92,144-149).
#include <fbgemm/FbgemmConvert.h>
#include <fbgemm/FbgemmEmbedding.h>

#include <algorithm>
#include <cstdint>
#include <functional>
#include <thread>
#include <vector>

namespace {

int64_t row_bytes(int ty, int D, int align) {
  int64_t u;
  switch (ty) {
    case 0: u = 4ll * D; break;
    case 1: u = 2ll * D; break;
    case 2: u = D + 4ll; break;
    case 3: u = D / 2 + 4ll; break;
    case 4: u = D / 4 + 4ll; break;
    case 6: u = D; break;
    default: return -1;
  }
  if (align > 1) u = (u + align - 1) / align * align;
  return u;
}

// Runs fn(t, b0, b1) over (table, bag-chunk) items on `nthreads` threads.
template <class F>
int parallel_bags(int T, int64_t B, int nthreads, F fn) {
  const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(256, B));
  const int64_t per_t = (B + chunk - 1) / chunk;
  const int64_t items = static_cast<int64_t>(T) * per_t;
  std::vector<int> rc(std::max(1, nthreads), 0);
  auto worker = [&](int w) {
    for (int64_t it = w; it < items; it += nthreads) {
      const int t = static_cast<int>(it / per_t);
      const int64_t b0 = (it % per_t) * chunk;
      const int64_t b1 = std::min(B, b0 + chunk);
      if (!fn(t, b0, b1)) rc[w] = -1;
    }
  };
  if (nthreads <= 1) {
    nthreads = 1;
    worker(0);
  } else {
    std::vector<std::thread> th;
    for (int w = 0; w < nthreads; ++w) th.emplace_back(worker, w);
    for (auto& x : th) x.join();
  }
  for (int v : rc)
    if (v) return v;
  return 0;
}

// offsets of bags [b0, b1] of table t rebased to the chunk's first index.
void rebase(const int64_t* offsets, int64_t base_bag, int64_t n, std::vector<int64_t>& out) {
  out.resize(n + 1);
  const int64_t s = offsets[base_bag];
  for (int64_t i = 0; i <= n; ++i) out[i] = offsets[base_bag + i] - s;
}

}  // namespace

extern "C" int fb_tbe_forward_f32(const float* W, const int64_t* w_off, const int32_t* D_off,
                                  int T, int64_t B, const int64_t* indices,
                                  const int64_t* offsets, int pooling, const float* iw,
                                  float* out, int64_t total_D, const int64_t* rows_per_table,
                                  int nthreads) {
  using K = fbgemm::EmbeddingSpMDMKernelSignature<float, int64_t, int64_t, float>::Type;
  std::vector<K> kern(T);
  for (int t = 0; t < T; ++t) {
    const int D = D_off[t + 1] - D_off[t];
    kern[t] = fbgemm::GenerateEmbeddingSpMDMWithStrides<float, int64_t, int64_t, float>(
        D, iw != nullptr, pooling == 1, 16, false, true, total_D, D);
  }
  return parallel_bags(T, B, nthreads, [&](int t, int64_t b0, int64_t b1) {
    std::vector<int64_t> off;
    rebase(offsets, t * B + b0, b1 - b0, off);
    const int64_t s = offsets[t * B + b0];
    return kern[t](b1 - b0, off.back(), rows_per_table[t], W + w_off[t], indices + s, off.data(),
                   iw ? iw + s : nullptr, out + b0 * total_D + D_off[t]);
  });
}

// fp16 weight rows (raw binary16 bits), fp32 output: the kernel fbgemm_gpu's
// CPU TBE forward uses for fp16 weights.
extern "C" int fb_tbe_forward_f16w(const uint16_t* W, const int64_t* w_off, const int32_t* D_off,
                                   int T, int64_t B, const int64_t* indices,
                                   const int64_t* offsets, int pooling, const float* iw,
                                   float* out, int64_t total_D, const int64_t* rows_per_table,
                                   int nthreads) {
  using K = fbgemm::EmbeddingSpMDMKernelSignature<uint16_t, int64_t, int64_t, float>::Type;
  std::vector<K> kern(T);
  for (int t = 0; t < T; ++t) {
    const int D = D_off[t + 1] - D_off[t];
    kern[t] = fbgemm::GenerateEmbeddingSpMDMWithStrides<uint16_t, int64_t, int64_t, float>(
        D, iw != nullptr, pooling == 1, 16, false, true, total_D, D);
  }
  return parallel_bags(T, B, nthreads, [&](int t, int64_t b0, int64_t b1) {
    std::vector<int64_t> off;
    rebase(offsets, t * B + b0, b1 - b0, off);
    const int64_t s = offsets[t * B + b0];
    return kern[t](b1 - b0, off.back(), rows_per_table[t], W + w_off[t], indices + s, off.data(),
                   iw ? iw + s : nullptr, out + b0 * total_D + D_off[t]);
  });
}

// FBGEMM's hfp8 conversions (FbgemmConvert.h:181-200), one value at a time.
extern "C" float fb_hfp8_to_float(uint8_t v, int ebits, int ebias) {
  float f;
  fbgemm::Float8ToFloat_ref(v, &f, ebits, ebias);
  return f;
}

extern "C" uint8_t fb_float_to_hfp8(float x, int ebits, int ebias) {
  uint8_t v;
  fbgemm::FloatToFloat8_ref(x, &v, ebits, ebias);
  return v;
}

extern "C" int fb_nbit_forward(const uint8_t* W, const int64_t* w_off, const uint8_t* tys,
                               const int32_t* D_off, int T, int64_t B, const int64_t* indices,
                               const int64_t* offsets, int pooling, const float* iw,
                               int row_align, int out_kind, void* out, int64_t total_D,
                               const int64_t* rows_per_table, int nthreads, int fp8_ebits,
                               int fp8_ebias) {
  if (out_kind != 1 && out_kind != 2) return -3;  // the harness serves fp16 and bf16 output
  const bool bf16 = out_kind == 2;
  using K8 = fbgemm::EmbeddingSpMDMKernelSignature<uint8_t, int64_t, int64_t, uint16_t>::Type;
  using K16 = fbgemm::EmbeddingSpMDMKernelSignature<uint16_t, int64_t, int64_t, uint16_t>::Type;
  using K32 = fbgemm::EmbeddingSpMDMKernelSignature<float, int64_t, int64_t, uint16_t>::Type;
  std::vector<K8> k8(T);
  std::vector<K16> k16(T);
  std::vector<K32> k32(T);
  for (int t = 0; t < T; ++t) {
    const int D = D_off[t + 1] - D_off[t];
    const int64_t stride = row_bytes(tys[t], D, row_align);
    if (stride < 0) return -1;
    const bool w = iw != nullptr, mean = pooling == 1;
    switch (tys[t]) {
      case 0:
        k32[t] = fbgemm::GenerateEmbeddingSpMDMWithStrides<float, int64_t, int64_t, uint16_t>(
            D, w, mean, 16, false, true, total_D, stride / 4, true, false, bf16);
        break;
      case 1:
        k16[t] = fbgemm::GenerateEmbeddingSpMDMWithStrides<uint16_t, int64_t, int64_t, uint16_t>(
            D, w, mean, 16, false, true, total_D, stride / 2, true, false, bf16);
        break;
      case 2:
        k8[t] = fbgemm::GenerateEmbeddingSpMDMWithStrides<uint8_t, int64_t, int64_t, uint16_t>(
            D, w, mean, 16, false, true, total_D, stride, /*scale_bias_last=*/false, false, bf16);
        break;
      case 3:
      case 4:
        k8[t] = fbgemm::GenerateEmbeddingSpMDMNBitWithStrides<int64_t, int64_t, uint16_t>(
            tys[t] == 3 ? 4 : 2, D, w, mean, 16, false, true, total_D, stride,
            /*scale_bias_last=*/false, bf16);
        break;
      case 6:  // weighted when the call passes weights
        k8[t] = fbgemm::GenerateEmbeddingSpMDMFP8WithStrides<int64_t, int64_t, uint16_t>(
            D, mean, false, true, total_D, stride, fp8_ebits, fp8_ebias, bf16);
        break;
      default:
        return -1;
    }
  }
  uint16_t* o = static_cast<uint16_t*>(out);
  return parallel_bags(T, B, nthreads, [&](int t, int64_t b0, int64_t b1) {
    std::vector<int64_t> off;
    rebase(offsets, t * B + b0, b1 - b0, off);
    const int64_t s = offsets[t * B + b0];
    const uint8_t* Wt = W + w_off[t];
    uint16_t* ot = o + b0 * total_D + D_off[t];
    const float* wt = iw ? iw + s : nullptr;
    switch (tys[t]) {
      case 0:
        return k32[t](b1 - b0, off.back(), rows_per_table[t], reinterpret_cast<const float*>(Wt),
                      indices + s, off.data(), wt, ot);
      case 1:
        return k16[t](b1 - b0, off.back(), rows_per_table[t],
                      reinterpret_cast<const uint16_t*>(Wt), indices + s, off.data(), wt, ot);
      default:
        return k8[t](b1 - b0, off.back(), rows_per_table[t], Wt, indices + s, off.data(), wt, ot);
    }
  });
}
