// The C ABI's host code under AddressSanitizer / UndefinedBehaviorSanitizer,
// with no GPU: the library's sources are compiled host-only (no device code)
// and linked into this driver by tests/test_host_model.py.  It checks
//   * every workspace-size function against a model of what the kernels
//     address (the persistent decode kernel: block offsets, shared-prefix
//     skips and header words [3B + 1] ints, piece slots -- two per row and
//     one per workgroup -- of (m, l) and D floats per query head, at up to
//     4 x the CU count workgroups; the
//     per-row kernel: one partial per 256-token partition; the prefix pass:
//     16 splits of (m, l) + D floats per row and head; the sampler: a
//     (maximum, sigma) pair per (row, 512-element segment)), over
//     batch sizes 1..7000, heads, head dims and table widths;
//   * that each entry point refuses bad arguments (null pointers, negative
//     or oversized counts, misaligned buffers, short workspaces) on the host
//     with the documented status, before anything is enqueued.
// No call here reaches a kernel launch.  Exit status 0 = all passed.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "litevllm_hip.h"

static int g_fail = 0;
#define CHECK(c, ...)                                               \
  do {                                                              \
    if (!(c)) {                                                     \
      if (g_fail < 30) {                                            \
        std::fprintf(stderr, "FAIL %s:%d ", __FILE__, __LINE__);    \
        std::fprintf(stderr, __VA_ARGS__);                          \
        std::fprintf(stderr, " [%s]\n", lv_last_error());           \
      }                                                             \
      ++g_fail;                                                     \
    }                                                               \
  } while (0)

static size_t a256(size_t x) { return (x + 255) / 256 * 256; }

// Bytes the decode kernels address for B decode rows (see the header).
static size_t decode_need(int B, int H, int D, int bs, int max_blocks, int cus) {
  // persistent kernel, worst case one kv head: 4 workgroups per CU
  const size_t wgs = (size_t)cus * 4;
  const size_t slots = 2 * (size_t)B + wgs;
  const size_t pers = a256(4 * (size_t)(3 * B + 1)) + a256(4 * 2 * slots * H) +
                      a256(4 * slots * H * D);
  // workgroup-per-row kernel (above 8 kv heads): 256-token partitions
  const size_t unit = 4 * (size_t)bs;
  const size_t part = (256 + unit - 1) / unit * unit;
  const size_t tokens = (size_t)max_blocks * bs;
  const size_t parts = (tokens + part - 1) / part;
  size_t rows = 0;
  if (parts > 1) rows = a256((size_t)B * H * parts * D * 4) + a256((size_t)B * H * parts * 2 * 4);
  return pers > rows ? pers : rows;
}

int main() {
  CHECK(lv_abi_version() == LV_ABI_VERSION, "abi version");
  const int cus = 256;   // without a device the library assumes 256 CUs (MI355X)

  // --- workspace sizes --------------------------------------------------
  const int batches[] = {1, 2, 3, 8, 16, 100, 256, 512, 4000, 7000};
  const int heads[] = {1, 8, 16, 32, 64};
  const int dims[] = {64, 128};
  const int widths[] = {1, 16, 128, 2560};
  for (int B : batches)
    for (int H : heads)
      for (int D : dims)
        for (int mb : widths) {
          const size_t ws = lv_paged_attention_workspace_size(B, B, B, H, D, 16, mb, 1, LV_BF16);
          CHECK(ws % 256 == 0 && ws >= decode_need(B, H, D, 16, mb, cus),
                "decode workspace B=%d H=%d D=%d mb=%d: %zu < %zu", B, H, D, mb, ws,
                decode_need(B, H, D, 16, mb, cus));
          // a prefill-only batch needs none
          CHECK(lv_paged_attention_workspace_size(B, 0, 4 * B, H, D, 16, mb, 4, LV_BF16) == 0,
                "no decode rows -> no workspace");
          const size_t n = (size_t)B * H * 16;
          CHECK(lv_paged_attention_prefix_workspace_size(B, H, D) ==
                    a256(n * 2 * 4) + a256(n * D * 4),
                "prefix workspace B=%d H=%d D=%d", B, H, D);
        }
  CHECK(lv_paged_attention_prefix_workspace_size(0, 16, 128) == 0, "empty prefix workspace");
  const int64_t vocabs[] = {1, 7, 511, 512, 513, 32000, 151936, 1 << 21};
  for (int64_t V : vocabs)
    for (int64_t B : {1, 40, 256, 1765, 4096}) {
      const int64_t nseg = (V + 511) / 512;      // (maximum, sigma) per (row, segment)
      const size_t want = (size_t)B * (size_t)(nseg * 8) + 256;
      CHECK(lv_sample_workspace_size(B, V) == want, "sampler workspace B=%lld V=%lld",
            (long long)B, (long long)V);
    }
  CHECK(lv_sample_workspace_size(0, 100) == 0 && lv_sample_workspace_size(4, 0) == 0 &&
            lv_sample_workspace_size(4, (1 << 21) + 1) == 0,
        "sampler workspace of empty / oversized calls");

  // --- argument checks (pointers below are never dereferenced) ----------
  void* p = (void*)0x1000;
  const int32_t* pi = (const int32_t*)0x1000;
  CHECK(lv_kv_scatter(nullptr, 8, nullptr, 8, nullptr, nullptr, nullptr, 4, 2, 4, 16, 10, LV_BF16,
                      nullptr) == LV_ERR_INVALID, "kv_scatter nulls");
  CHECK(lv_kv_scatter(nullptr, 0, nullptr, 0, nullptr, nullptr, nullptr, 0, 1, 1, 1, 1, LV_F32,
                      nullptr) == LV_OK, "kv_scatter empty");
  CHECK(lv_kv_scatter(p, 8, p, 8, p, p, (const int64_t*)p, -1, 2, 4, 16, 10, LV_BF16, nullptr) ==
            LV_ERR_INVALID, "kv_scatter negative count");
  CHECK(lv_pack_inputs(nullptr, 0, nullptr, 0, nullptr, 0, nullptr, 0, 0, 16, 0, nullptr, nullptr,
                       nullptr, nullptr, nullptr, nullptr, nullptr, nullptr) == LV_ERR_INVALID,
        "pack zero sequences");
  CHECK(lv_pack_inputs((const lv_seq_desc*)p, -3, pi, 4, (const int64_t*)p, 4, nullptr, 0, 4, 16, 4,
                       (int64_t*)p, (int64_t*)p, (int64_t*)p, (int32_t*)p, (int32_t*)p,
                       (int32_t*)p, (int32_t*)p, nullptr) == LV_ERR_INVALID,
        "pack negative sequences");
  CHECK(lv_paged_attention(nullptr, 0, nullptr, nullptr, 1, nullptr, 1, nullptr, nullptr, 2, 3, 2,
                           1, 16, 8, 128, 16, 0.1f, nullptr, 0, nullptr, 0, LV_BF16, nullptr) ==
            LV_ERR_INVALID, "attention num_decodes > num_seqs");
  CHECK(lv_paged_attention(p, 2048, p, p, 100, pi, 16, nullptr, pi, 4, 4, 4, 1, 16, 6, 128, 16,
                           0.1f, p, 2048, p, 1 << 20, LV_BF16, nullptr) == LV_ERR_INVALID,
        "attention heads not a multiple of kv heads");
  CHECK(lv_paged_attention(p, 2048, p, p, 100, pi, 16, nullptr, pi, 4, 2, 4, 1, 16, 8, 128, 16,
                           0.1f, p, 2048, p, 1 << 20, LV_BF16, nullptr) == LV_ERR_INVALID,
        "attention chunks without cu_seqlens");
  CHECK(lv_paged_attention((void*)0x1004, 2048, p, p, 100, pi, 16, nullptr, pi, 4, 4, 4, 1, 16, 8,
                           128, 16, 0.1f, p, 2048, p, 1 << 20, LV_BF16, nullptr) == LV_ERR_INVALID,
        "attention misaligned query");
  CHECK(lv_paged_attention(p, 2048, p, p, 100, pi, 1 << 22, nullptr, pi, 4, 4, 4, 1, 16, 8, 128,
                           16, 0.1f, p, 2048, p, 1 << 20, LV_BF16, nullptr) == LV_ERR_INVALID,
        "attention table too wide");
  CHECK(lv_paged_attention(p, 2048, p, p, 100, pi, 16, nullptr, pi, 4, 4, 4, 1, 16, 8, 128, 16,
                           0.1f, p, 2048, p, 255, LV_BF16, nullptr) == LV_ERR_WORKSPACE,
        "attention short workspace");
  CHECK(lv_paged_attention_prefix(nullptr, 0, nullptr, nullptr, 1, nullptr, 1, nullptr, nullptr, 8,
                                  8, 8, 1, 16, 8, 128, 16, 0.1f, nullptr, 0, nullptr, 0, pi, pi, 4,
                                  pi, -1, p, 1 << 30, LV_BF16, nullptr) == LV_ERR_INVALID,
        "prefix negative num_members");
  CHECK(lv_paged_attention_prefix(nullptr, 0, nullptr, nullptr, 1, nullptr, 1, nullptr, nullptr, 8,
                                  8, 8, 1, 16, 8, 128, 16, 0.1f, nullptr, 0, nullptr, 0, pi,
                                  (const int32_t*)0x1004, 4, pi, 8, p, 1 << 30, LV_BF16,
                                  nullptr) == LV_ERR_INVALID,
        "prefix misaligned items");
  CHECK(lv_paged_attention_prefix(nullptr, 0, nullptr, nullptr, 1, nullptr, 1, nullptr, nullptr, 8,
                                  8, 8, 1, 16, 8, 128, 16, 0.1f, nullptr, 0, nullptr, 0, pi, pi, 4,
                                  pi, 8, p, 16, LV_BF16, nullptr) == LV_ERR_WORKSPACE,
        "prefix short workspace");
  CHECK(lv_sample(nullptr, 4, 0, 0, nullptr, nullptr, nullptr, nullptr, 0, LV_BF16, nullptr) ==
            LV_ERR_INVALID, "sample zero vocab");
  CHECK(lv_sample(p, 4, 1000, 999, (const float*)p, (const float*)p, (int64_t*)p, p, 1 << 20,
                  LV_BF16, nullptr) == LV_ERR_INVALID, "sample stride < vocab");
  CHECK(lv_sample(p, 4, 1000, 1000, (const float*)p, nullptr, (int64_t*)p, p, 1 << 20, LV_BF16,
                  nullptr) == LV_ERR_INVALID, "sample without uniforms");
  CHECK(lv_sample(p, 4, 1000, 1000, (const float*)p, (const float*)p, (int64_t*)p, p, 8, LV_BF16,
                  nullptr) == LV_ERR_WORKSPACE, "sample short workspace");
  CHECK(lv_sample(p, 0, 1000, 1000, nullptr, nullptr, nullptr, nullptr, 0, LV_BF16, nullptr) ==
            LV_OK, "sample empty batch");
  CHECK(lv_sample_noalloc(p, 4096, 151936, 151936, (const float*)p, (const float*)p, (int64_t*)p,
                          LV_BF16, nullptr) == LV_ERR_WORKSPACE, "noalloc beyond its scratch");
  CHECK(lv_sample_noalloc(nullptr, 4, 100, 100, nullptr, nullptr, nullptr, LV_BF16, nullptr) ==
            LV_ERR_INVALID, "noalloc nulls");
  CHECK(lv_add_rms_norm(nullptr, 0, nullptr, 0, nullptr, nullptr, 0, 4, 1024, 1e-6f, LV_BF16,
                        nullptr) == LV_ERR_INVALID, "rms norm nulls");
  CHECK(lv_silu_mul(nullptr, 0, nullptr, 0, 4, 3072, LV_BF16, nullptr) == LV_ERR_INVALID,
        "silu_mul nulls");
  CHECK(lv_linear_supported(256, 1024, 1000, LV_ACT_NONE, LV_BF16) == 0,
        "linear: k not a multiple of 128");
  if (g_fail) {
    std::fprintf(stderr, "%d checks failed\n", g_fail);
    return 1;
  }
  std::printf("C ABI host checks: all passed\n");
  return 0;
}
