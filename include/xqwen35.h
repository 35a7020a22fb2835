/* xqwen35.h - the public C ABI of the decode library, byte-compatible with the
 * reference's customlib/include/xqwen35.h (status codes :21-28, xq_options
 * :30-40, xq_metrics :42-58, the entry points :60-77), so an existing caller
 * (benchmark harness, quality runner, tests) links against this library
 * unchanged.  Behind it, the model runs device-resident on an MI355X through
 * the hand-written gfx950 kernels of libxqhip.so.
 */
#ifndef XQWEN35_H_
#define XQWEN35_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XQ_API __attribute__((visibility("default")))

typedef struct xq_session xq_session;

typedef enum xq_status {
    XQ_OK = 0,
    XQ_ERR_INVALID_ARGUMENT = -1,
    XQ_ERR_NOT_READY = -2,
    XQ_ERR_MODEL = -3,
    XQ_ERR_RUNTIME = -4,
    XQ_ERR_BUFFER_TOO_SMALL = -5
} xq_status;

typedef struct xq_options {
    size_t struct_size;
    const char* backend;
    int threads;
    int quant_bits;
    int group_size;
    int max_context_tokens;
    int enable_autotune;
    int use_mnn_fallback;
    const char* telemetry_path;
} xq_options;

typedef struct xq_metrics {
    size_t struct_size;
    uint64_t prompt_tokens;
    uint64_t generated_tokens;
    double load_ms;
    double prefill_ms;
    double first_token_ms;
    double decode_total_ms;
    double total_generate_ms;
    double prefill_tokens_per_second;
    double decode_tokens_per_second;
    uint64_t rss_kb;
    uint64_t pss_kb;
    char backend[64];
    char selected_kernels[512];
    char error[256];
} xq_metrics;

/* Replaces xq_create (customlib/runtime/session.cpp:620-632). */
XQ_API xq_status xq_create(const char* model_dir, const xq_options* options, xq_session** out_session);
/* Replaces xq_destroy (session.cpp:634-636). */
XQ_API void xq_destroy(xq_session* session);
/* Replaces xq_prefill -> Session::prefill (session.cpp:304-342, 638-643). */
XQ_API xq_status xq_prefill(xq_session* session, const int32_t* token_ids, size_t n_tokens, xq_metrics* out_metrics);
/* Replaces xq_decode_one -> Session::decodeOne (session.cpp:344-383, 645-650). */
XQ_API xq_status xq_decode_one(xq_session* session, int32_t* out_token_id, xq_metrics* out_metrics);
/* Replaces xq_generate -> Session::generate (session.cpp:385-421, 652-664). */
XQ_API xq_status xq_generate(xq_session* session,
                             const int32_t* token_ids,
                             size_t n_tokens,
                             size_t max_new_tokens,
                             int32_t* output_buffer,
                             size_t output_capacity,
                             xq_metrics* out_metrics);
/* Replaces xq_reset -> Session::reset (session.cpp:505-525). */
XQ_API xq_status xq_reset(xq_session* session);
/* Replaces xq_get_last_metrics (session.cpp:527-530). */
XQ_API xq_status xq_get_last_metrics(xq_session* session, xq_metrics* out_metrics);
/* Replaces xq_get_backend_info (session.cpp:532-554). */
XQ_API xq_status xq_get_backend_info(xq_session* session, char* json_out, size_t json_capacity);
/* Replaces xq_get_kernel_trace_json (session.cpp:556-566). */
XQ_API xq_status xq_get_kernel_trace_json(xq_session* session, char* json_out, size_t json_capacity);
/* Replaces xq_get_debug_json (session.cpp:568-578, custom_model.cpp:1382-1436). */
XQ_API xq_status xq_get_debug_json(xq_session* session, char* json_out, size_t json_capacity);
/* Replaces xq_get_hidden_state (session.cpp:580-585, custom_model.cpp:1438-1447). */
XQ_API xq_status xq_get_hidden_state(xq_session* session, float* out_values, size_t value_capacity, size_t* out_size);
/* Replaces xq_run_vulkan_w4a16_selftest (session.cpp:708-710, vulkan_backend.cpp:1638-2029):
 * the same deterministic GEMV self-test, run on the HIP device. */
XQ_API xq_status xq_run_vulkan_w4a16_selftest(char* json_out, size_t json_capacity);

#ifdef __cplusplus
}
#endif

#endif /* XQWEN35_H_ */
