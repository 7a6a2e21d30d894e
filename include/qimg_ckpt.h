/* qimg_ckpt.h — C ABI of the quantized checkpoint format (libqimg_host.so).
 *
 * Files are safetensors: an 8-byte little-endian header length, a JSON
 * header, then the tensors back to back. A quantized linear "<name>" is
 * stored as I8 (int8) or F8_E4M3 (e4m3) [N, K] bytes of the Hadamard-rotated
 * weight plus "<name>.__scales__" F32 [N]; its Hadamard block is K & -K.
 * Functions return 0 (or a non-negative result) on success and -1 on
 * failure; where `err` is given, it receives a NUL-terminated message of at
 * most err_len bytes.
 */
#ifndef QIMG_CKPT_H
#define QIMG_CKPT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* SafeTensorsWriter (safetensors_writer.h:12-104): tensors are written in
 * the order they were added, the header padded with spaces to a multiple
 * of 8 bytes; the bytes equal the reference writer's for the same adds.
 * dtype is the header string ("I8", "F8_E4M3", "F32", "BF16", ...). */
void* qimg_st_writer_new(void);
int qimg_st_writer_add(void* writer, const char* name, const char* dtype, const int64_t* shape, int ndim,
                       const void* data, size_t nbytes);
int qimg_st_writer_write(void* writer, const char* path);
void qimg_st_writer_free(void* writer);

/* Quantization mode of a transformer checkpoint (transformer.h:146-156,
 * probing transformer_blocks.0.attn.to_q.weight): 0 = BF16 (quantized at
 * load), 1 = pre-quantized int8 (I8), 2 = pre-quantized e4m3 (F8_E4M3).
 * `path` is a .safetensors file or a directory as load_model_dir
 * (safetensors.h:235-274) takes it. -1 for an unreadable or malformed
 * checkpoint, including a tensor of unknown dtype (which the reference
 * skips with a message, safetensors.h:94-96). */
int qimg_checkpoint_kind(const char* path, char* err, int err_len);

/* The offline quantizer (quantize.cu:110-161, 334-341, 462-539): reads the
 * BF16 checkpoint at in_path, quantizes the linear weights of the
 * timestep embedder and of `num_blocks` transformer blocks (the reference
 * runs 60) with the Hadamard + per-row quantization of
 * qimg_quantize_weight on the current HIP device (mode
 * QIMG_QM_INT8_HADAMARD -> I8, QIMG_QM_FP8_HADAMARD -> F8_E4M3), copies the
 * biases, norms and boundary layers (F32 kept F32, other dtypes labelled
 * BF16, as the reference's passthrough), and writes out_path with the
 * reference's tensor order. Fails when a listed tensor is missing or a
 * quantized one is not a 2-D BF16 weight. */
int qimg_quantize_checkpoint(const char* in_path, const char* out_path, int mode, int num_blocks, char* err,
                             int err_len);

#ifdef __cplusplus
}
#endif

#endif /* QIMG_CKPT_H */
