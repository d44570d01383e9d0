/*
 * glacier_lora_file.h -- the 'LORA' v1 adapter binary (adapter_model.bin) in
 * libglacier_attn.so: write a set of adapter tensors, and read them back
 * with the reference's validation, so that adapters trained through this
 * library can be checkpointed, resumed and compared (host memory; copy to
 * the device with hipMemcpy).
 *
 * Layout (little-endian), as GgufLoraModel.SaveAdapter writes it
 * (src/Glacier.Tune/Model/GgufLoraModel.cs:636-650) and TuneBlockSerialization
 * .WriteTensor (src/Glacier.Tune/Model/ITuneBlock.cs:43-50) per tensor:
 *   uint32 magic 0x41524F4C ('LORA'), uint32 version 1, int32 layer_count,
 *   int32 rank, float32 alpha, int32 tensor_count, then tensor_count records
 *   of: name (a .NET BinaryWriter string: the UTF-8 byte count as a 7-bit
 *   varint, then the bytes), int32 dim0, int32 dim1, dim0 * dim1 float32
 *   row-major.  Names are "blk.<layer>.<proj>.lora_a.weight" / "lora_b"
 *   (ITuneBlock.cs:29-34; proj = attn_q, attn_k, attn_v, attn_qkv,
 *   attn_output, ffn_gate, ffn_up, ffn_down), A [in][rank] and B [rank][out]
 *   in the native layout, [rank][in] / [out][rank] in the PEFT one.
 * Reading follows GgufLoraModel.LoadAdapter (:697-796): a directory path
 * means <dir>/adapter_model.bin; bad magic, another version, a negative
 * tensor count, a non-finite or non-positive alpha with rank > 0, a
 * non-positive dimension and a truncated record are rejected with
 * GLACIER_LORA_ERR_DATA (the reference's InvalidDataException); a missing
 * file also gives GLACIER_LORA_ERR_DATA (FileNotFoundException).  Matching
 * names and shapes to a model (FindTargetTensor, :798-835) is the caller's:
 * glacier_lora_read can transpose a record to the other layout.
 */
#ifndef GLACIER_LORA_FILE_H
#define GLACIER_LORA_FILE_H

#include "glacier_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A file is missing, truncated or malformed. */
#define GLACIER_LORA_ERR_DATA 5

#define GLACIER_LORA_MAGIC 0x41524F4Cu
#define GLACIER_LORA_VERSION 1u

typedef struct glacier_lora_header {
  uint32_t version;
  int32_t layer_count;
  int32_t rank;
  float alpha;
  int32_t tensor_count;
} glacier_lora_header;

typedef struct glacier_lora_reader glacier_lora_reader;

/* Writes the file: n_tensors records of names[i], dims dim0[i] x dim1[i] and
 * host fp32 data[i] (row-major).  The file is written whole to a temporary
 * name beside path, then renamed over it. */
int glacier_lora_save(const char *path, int32_t layer_count, int32_t rank, float alpha,
                      int32_t n_tensors, const char *const *names, const int32_t *dim0,
                      const int32_t *dim1, const float *const *data);

/* Opens path (or path/adapter_model.bin), checks the header and returns it. */
int glacier_lora_open(const char *path, glacier_lora_header *header, glacier_lora_reader **reader);

/* The next record's name (NUL-terminated; name_cap must fit it) and dims.
 * Each record must then be consumed with glacier_lora_read before the next
 * call.  INVALID_ARGUMENT after the last record.  A name_cap too small for
 * the name gives INVALID_ARGUMENT with the needed size in the error text and
 * leaves the reader at the record's start, so a retry with a larger buffer
 * reads the same record.  A malformed or truncated record gives
 * GLACIER_LORA_ERR_DATA, and so does every later next/read on the reader. */
int glacier_lora_next(glacier_lora_reader *reader, char *name, int32_t name_cap, int32_t *dim0,
                      int32_t *dim1);

/* The current record's payload into dst: as stored ([dim0][dim1]), or with
 * transpose != 0 as [dim1][dim0] (the other layout, LoadAdapter :760-772).
 * dst NULL skips the record. */
int glacier_lora_read(glacier_lora_reader *reader, float *dst, int32_t transpose);

void glacier_lora_close(glacier_lora_reader *reader);

#ifdef __cplusplus
}
#endif

#endif /* GLACIER_LORA_FILE_H */
