// Host-side helpers: device properties, occupancy-sized persistent grids and
// the list of exported C-ABI symbols.
#include "tf_host.hpp"

#include <mutex>
#include <unordered_map>

#include "taraference_hip.h"

namespace {
std::mutex g_mu;
int g_cus[64];

struct OccKey {
    const void* fn;
    int threads, lds, dev;
    bool operator==(const OccKey& o) const {
        return fn == o.fn && threads == o.threads && lds == o.lds && dev == o.dev;
    }
};
struct OccHash {
    size_t operator()(const OccKey& k) const {
        return std::hash<const void*>()(k.fn) ^ ((size_t)k.threads << 40) ^
               ((size_t)k.lds << 12) ^ (size_t)k.dev;
    }
};
std::unordered_map<OccKey, int, OccHash> g_occ;
}  // namespace

int tf_device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_cus[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                hipSuccess || cus <= 0)
            cus = 256;
        g_cus[dev] = cus;
    }
    return g_cus[dev];
}

int tf_block_threads(int max_threads, long long tasks) {
    const long long cus = tf_device_cus();
    const long long waves_per_cu = (tasks + cus - 1) / cus;
    long long threads = ((waves_per_cu + 3) / 4) * 256;
    if (threads < 256) threads = 256;
    if (threads > max_threads) threads = max_threads;
    return (int)threads;
}

int tf_persistent_blocks(const void* kernel, int threads, int lds_bytes, int tasks) {
    if (tasks <= 0) return 1;
    const int cus = tf_device_cus();
    int dev = 0;
    (void)hipGetDevice(&dev);
    int per_cu = 0;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        OccKey key{kernel, threads, lds_bytes, dev};
        auto it = g_occ.find(key);
        if (it != g_occ.end()) {
            per_cu = it->second;
        } else {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads,
                                                             lds_bytes) != hipSuccess ||
                per_cu <= 0)
                per_cu = 1;
            g_occ[key] = per_cu;
        }
    }
    // every resident slot, but no workgroup without a task for each wave
    // (tasks are dealt out block-major, so the blocks share them evenly)
    const int waves_per_block = threads / 64;
    const long long max_blocks = (long long)cus * per_cu;
    const long long needed = (tasks + waves_per_block - 1) / waves_per_block;
    return (int)(needed < max_blocks ? needed : max_blocks);
}

static const char* const k_symbols[] = {
    "tf_version",
    "tf_exported_symbol_count",
    "tf_exported_symbol",
    "tf_quantize_q8",
    "tf_gemv_q4k_q8",
    "tf_gemv_q4k_q8_splitk",
    "tf_gemv_splitk_reduce",
    "tf_gemv_q4k_pair",
    "tf_gemv_q4k_dual",
    "tf_gemv_q4k_ffn",
    "tf_gemv_q4k_ffn_f32",
    "tf_gemv_q4k_f32",
    "tf_gemv_q4k_qkv",
    "tf_gemv_q6k_compact_q8",
    "tf_gemv_q6k_down_splitk",
    "tf_gemv_q6k_compact_q8_splitk",
    "tf_gemv_q6k_f32",
    "tf_q6k_compact_repack",
    "tf_gemv_q8_0_q8",
    "tf_gemv_q8_0_f32",
    "tf_gemv_q8_0_q8_splitk",
    "tf_gemv_q8_0_f32_splitk",
    "tf_gemv_q5_0_f32",
    "tf_gemv_q5_0_f32_splitk",
    "tf_gemv_q5_0_qk",
    "tf_gemv_q5_0_qkv",
    "tf_gemv_q8_0_qkv",
    "tf_gemm_q4k_f32",
    "tf_gemm_q6k_f32",
    "tf_attn_prefill",
    "tf_attn_prefill_d",
    "tf_flash_decode_partial",
    "tf_flash_decode_partial_d",
    "tf_flash_decode_reduce",
    "tf_flash_decode_n_split",
    "tf_fused_norm_qkv_rope_kv",
    "tf_fused_qkv_rope_kv",
    "tf_norm_quant",
    "tf_flash_decode_reduce_q8",
    "tf_flash_decode",
    "tf_flash_decode_noalloc",
    "tf_gemv_q4k_flash_out",
    "tf_gemv_q6k_q8_argmax",
    "tf_gemv_q4k_ffn_norm",
    "tf_gemv_q6k_compact_f32",
    "tf_gemv_q6k_head_argmax",
    "tf_argmax_key_finalize",
    "tf_embed_row",
    "tf_rms_norm",
    "tf_rope_neox",
    "tf_copy_kv_f16",
    "tf_argmax",
    "tf_gguf_open",
    "tf_gguf_close",
    "tf_gguf_version",
    "tf_gguf_data_offset",
    "tf_gguf_file_size",
    "tf_gguf_n_tensors",
    "tf_gguf_tensor_at",
    "tf_gguf_find_tensor",
    "tf_gguf_meta_type",
    "tf_gguf_meta_u32",
    "tf_gguf_meta_u64",
    "tf_gguf_meta_f32",
    "tf_gguf_meta_str",
    "tf_gguf_meta_bool",
    "tf_gguf_meta_i64",
    "tf_gguf_meta_f64",
    "tf_gguf_meta_array",
    "tf_gguf_meta_array_str",
    "tf_gguf_meta_array_f64",
    "tf_ggml_block_size",
    "tf_ggml_type_size",
    "tf_ggml_nbytes",
    "tf_gguf_model_config",
    "tf_model_create",
    "tf_model_destroy",
    "tf_model_forward",
    "tf_model_generate",
    "tf_model_prefill",
    "tf_model_set_path",
    "tf_model_get_path",
    "tf_model_logits",
    "tf_model_keep_stage_vectors",
    "tf_model_stage_vector",
    "tf_model_q8_record",
    "tf_decode_step_quantize_q8",
    "tf_stream_read_probe",
    "tf_model_k_cache",
    "tf_model_v_cache",
    "tf_q4k_block_dots",
    "tf_q6k_block_dots",
};

extern "C" int tf_version(void) { return 100; }
extern "C" int tf_exported_symbol_count(void) {
    return (int)(sizeof(k_symbols) / sizeof(k_symbols[0]));
}
extern "C" const char* tf_exported_symbol(int i) {
    if (i < 0 || i >= tf_exported_symbol_count()) return nullptr;
    return k_symbols[i];
}

int tf_set_lds_limit(const void* kernel, int bytes) {
    static std::mutex mu;
    static std::unordered_map<const void*, int> done[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(mu);
    int& have = done[dev][kernel];
    if (have >= bytes) return 0;
    const hipError_t rc =
        hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (rc != hipSuccess) return (int)rc;
    have = bytes;
    return 0;
}
