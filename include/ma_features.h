/*
 * ma_features.h -- C-ABI of the GPU tick-feature pass (libma_attn.so).
 *
 * Replaces the host-side preprocessing of the reference's TickDataset
 * (/root/reference src/data_loader.py:15-28): microstructure features of raw
 * ticks, z-scored per column, as float32 rows [n, 5] in the order
 * [price, bid_ask_spread, wap, order_book_imbalance, time_diff].
 */
#ifndef MA_FEATURES_H
#define MA_FEATURES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of device workspace ma_tick_features needs for n ticks. */
size_t ma_tick_features_workspace_size(int64_t n);

/*
 * Device float64 columns of n ticks -> out: device float32 [n, 5];
 * stats: device float64 [10] = 5 column means then 5 sample standard
 * deviations (ddof 1, as pandas' std).  Asynchronous on `stream`
 * (hipStream_t); allocates nothing.  Returns non-zero (ma_attn_last_error())
 * on invalid arguments.
 */
int ma_tick_features(const double* timestamp, const double* price, const double* bid_price,
                     const double* ask_price, const double* bid_volume, const double* ask_volume,
                     int64_t n, float* out, double* stats, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * ma_tick_features with caller-created HIP events (hipEvent_t, either may be
 * NULL) stamped on the pass's first kernel start and last kernel end
 * (hipExtLaunchKernel), as ma_attn_forward_timed.  For timing; no
 * counterpart in the reference.
 */
int ma_tick_features_timed(const double* timestamp, const double* price, const double* bid_price,
                           const double* ask_price, const double* bid_volume, const double* ask_volume,
                           int64_t n, float* out, double* stats, void* workspace, size_t workspace_bytes,
                           void* stream, void* start_event, void* stop_event);

#ifdef __cplusplus
}
#endif

#endif /* MA_FEATURES_H */
