// A C++ host program that uses libswattn.so through its C ABI alone (no
// Python, no torch): router-mask compaction, the routed prefill forward and
// its backward, on device buffers it allocates with the HIP runtime.  It is
// the caller a non-Python host would write against include/swattn.h, and
// tests/test_gpu_c_abi_caller.py checks what it writes against the oracle.
//
//   prefill_caller IN OUT
//
// IN:  int64 header {batch, seq_q, seq_kv, heads_q, heads_kv, window}, then
//      q (batch*seq_q*heads_q*128 bf16), k and v (batch*seq_kv*heads_kv*128
//      bf16 each), dout (like q), mask (batch*seq_q bytes, nonzero = full).
// OUT: int64 nf, the full list (nf int32), the local list (n - nf int32),
//      O (bf16 like q), LSE (batch*seq_q*heads_q fp32), dq, dk, dv (bf16).
// Exit status 0 on success; otherwise the failing call and
// swattn_last_error() go to stderr.

#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>

#include <cmath>
#include <vector>

#include "swattn.h"

namespace {

bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return false;
}

bool sw_ok(int st, const char* what) {
  if (st == 0) return true;
  fprintf(stderr, "%s: status %d: %s\n", what, st, swattn_last_error());
  return false;
}

// Device buffer freed on scope exit.
struct DevBuf {
  void* p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  bool alloc(size_t bytes, const char* what) {
    return hip_ok(hipMalloc(&p, bytes > 0 ? bytes : 1), what);
  }
};

template <class T>
bool read_vec(FILE* f, std::vector<T>& v, size_t n) {
  v.resize(n);
  return n == 0 || fread(v.data(), sizeof(T), n, f) == n;
}

template <class T>
bool write_vec(FILE* f, const std::vector<T>& v) {
  return v.empty() || fwrite(v.data(), sizeof(T), v.size(), f) == v.size();
}

template <class T>
bool to_host(std::vector<T>& h, const DevBuf& d, size_t n, const char* what) {
  h.resize(n);
  return n == 0 || hip_ok(hipMemcpy(h.data(), d.p, n * sizeof(T), hipMemcpyDeviceToHost), what);
}

template <class T>
bool to_device(DevBuf& d, const std::vector<T>& h, const char* what) {
  if (!d.alloc(h.size() * sizeof(T), what)) return false;
  return h.empty() ||
         hip_ok(hipMemcpy(d.p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), what);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    fprintf(stderr, "usage: %s IN OUT\n", argv[0]);
    return 2;
  }
  FILE* in = fopen(argv[1], "rb");
  if (!in) {
    fprintf(stderr, "cannot open %s\n", argv[1]);
    return 2;
  }
  int64_t hdr[6];
  if (fread(hdr, sizeof(int64_t), 6, in) != 6) {
    fprintf(stderr, "short header\n");
    return 2;
  }
  const int32_t batch = static_cast<int32_t>(hdr[0]);
  const int64_t seq_q = hdr[1], seq_kv = hdr[2];
  const int32_t hq = static_cast<int32_t>(hdr[3]), hkv = static_cast<int32_t>(hdr[4]);
  const int32_t window = static_cast<int32_t>(hdr[5]);
  const int32_t d = 128;
  const size_t nq = static_cast<size_t>(batch) * seq_q * hq * d;
  const size_t nkv = static_cast<size_t>(batch) * seq_kv * hkv * d;
  const int64_t n = static_cast<int64_t>(batch) * seq_q;
  std::vector<uint16_t> q, k, v, dout;
  std::vector<uint8_t> mask;
  const bool got = read_vec(in, q, nq) && read_vec(in, k, nkv) && read_vec(in, v, nkv) &&
                   read_vec(in, dout, nq) && read_vec(in, mask, static_cast<size_t>(n));
  fclose(in);
  if (!got) {
    fprintf(stderr, "short input\n");
    return 2;
  }
  printf("prefill_caller: B%d S%lld Skv%lld Hq%d/Hkv%d W%d, library version %d\n", batch,
         static_cast<long long>(seq_q), static_cast<long long>(seq_kv), hq, hkv, window,
         swattn_version());
  fflush(stdout);

  hipStream_t stream = nullptr;
  if (!hip_ok(hipStreamCreate(&stream), "hipStreamCreate")) return 1;
  DevBuf dq_, dk_, dv_, dout_d, q_d, k_d, v_d, mask_d, idx_d, cnt_d, cws, o_d, lse_d, fws, bws;
  if (!to_device(q_d, q, "q") || !to_device(k_d, k, "k") || !to_device(v_d, v, "v") ||
      !to_device(dout_d, dout, "dout") || !to_device(mask_d, mask, "mask"))
    return 1;

  // Compaction (build_switch_query_indices): one small read of the split point.
  const size_t cws_bytes = swattn_compact_workspace_bytes(n);
  if (!idx_d.alloc(n * sizeof(int32_t), "indices") || !cnt_d.alloc(2 * sizeof(int32_t), "counts") ||
      !cws.alloc(cws_bytes, "compact workspace"))
    return 1;
  if (!sw_ok(swattn_compact(static_cast<const uint8_t*>(mask_d.p), n,
                            static_cast<int32_t*>(idx_d.p), static_cast<int32_t*>(cnt_d.p), cws.p,
                            cws_bytes, stream),
             "swattn_compact"))
    return 1;
  int32_t counts[2] = {0, 0};
  if (!hip_ok(hipMemcpyAsync(counts, cnt_d.p, sizeof(counts), hipMemcpyDeviceToHost, stream),
              "counts") ||
      !hip_ok(hipStreamSynchronize(stream), "sync"))
    return 1;
  const int64_t nf = counts[0], nl = counts[1];
  const int32_t* full = static_cast<const int32_t*>(idx_d.p);
  const int32_t* local = full + nf;

  // Forward, with the workspace that allows the key-range split.
  const float scale_log2 = static_cast<float>(1.0 / std::sqrt(128.0) * 1.4426950408889634);
  const size_t fws_bytes =
      swattn_prefill_split_workspace_bytes(batch, seq_q, seq_kv, hq, hkv, d, window, nf, nl);
  if (fws_bytes == 0) {
    fprintf(stderr, "unsupported shape\n");
    return 1;
  }
  if (!o_d.alloc(nq * sizeof(uint16_t), "out") ||
      !lse_d.alloc(static_cast<size_t>(n) * hq * sizeof(float), "lse") ||
      !fws.alloc(fws_bytes, "forward workspace"))
    return 1;
  if (!sw_ok(swattn_prefill_fwd(q_d.p, k_d.p, v_d.p, full, nf, local, nl, nullptr, nullptr,
                                nullptr, o_d.p, static_cast<float*>(lse_d.p), batch, seq_q,
                                seq_kv, hq, hkv, d, window, scale_log2, fws.p, fws_bytes, stream),
             "swattn_prefill_fwd"))
    return 1;

  // Backward (the lists cover every position, so every dq row is written).
  const size_t bws_bytes = swattn_prefill_bwd_workspace_bytes(batch, seq_kv, hq, hkv, d, window,
                                                              nf, nl);
  if (!dq_.alloc(nq * sizeof(uint16_t), "dq") || !dk_.alloc(nkv * sizeof(uint16_t), "dk") ||
      !dv_.alloc(nkv * sizeof(uint16_t), "dv") || !bws.alloc(bws_bytes, "backward workspace"))
    return 1;
  if (!sw_ok(swattn_prefill_bwd(q_d.p, k_d.p, v_d.p, o_d.p, static_cast<const float*>(lse_d.p),
                                dout_d.p, full, nf, local, nl, nullptr, nullptr, nullptr, dq_.p,
                                dk_.p, dv_.p, batch, seq_q, seq_kv, hq, hkv, d, window,
                                scale_log2, bws.p, bws_bytes, stream),
             "swattn_prefill_bwd"))
    return 1;
  if (!hip_ok(hipStreamSynchronize(stream), "sync")) return 1;

  std::vector<int32_t> idx;
  std::vector<uint16_t> o, dq, dk, dv;
  std::vector<float> lse;
  if (!to_host(idx, idx_d, static_cast<size_t>(n), "indices") || !to_host(o, o_d, nq, "out") ||
      !to_host(lse, lse_d, static_cast<size_t>(n) * hq, "lse") || !to_host(dq, dq_, nq, "dq") ||
      !to_host(dk, dk_, nkv, "dk") || !to_host(dv, dv_, nkv, "dv"))
    return 1;
  (void)hipStreamDestroy(stream);

  FILE* out = fopen(argv[2], "wb");
  if (!out) {
    fprintf(stderr, "cannot open %s\n", argv[2]);
    return 2;
  }
  const bool put = fwrite(&nf, sizeof(nf), 1, out) == 1 && write_vec(out, idx) &&
                   write_vec(out, o) && write_vec(out, lse) && write_vec(out, dq) &&
                   write_vec(out, dk) && write_vec(out, dv);
  fclose(out);
  if (!put) {
    fprintf(stderr, "short write\n");
    return 2;
  }
  printf("prefill_caller: %lld full, %lld local rows; wrote %s\n", static_cast<long long>(nf),
         static_cast<long long>(nl), argv[2]);
  return 0;
}
