/*
 * settings.c - the library's environment switches, read once.
 *
 * The kernels' tile overrides and graph_eval's fold switches used to be
 * read with getenv on every launch: a few hundred nanoseconds per call,
 * and a data race with any thread calling setenv. They are now parsed
 * once, on first use, into one immutable snapshot. A caller that changes
 * the environment afterwards (tests toggling a fold) calls
 * sam3_hip_reload_settings(), which publishes a new snapshot; launches
 * already running keep reading the one they started with.
 *
 * Every switch defaults to the production behaviour when unset.
 */
#include "sam3_hip.h"
#include "sam3_hip_internal.h"
#include "s3k.h"

#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>

static int env_int(const char *name, int dflt)
{
	const char *s = getenv(name);
	if (!s || !*s)
		return dflt;
	return (int)strtol(s, NULL, 10);
}

/* A switch that is on unless set to 0. */
static int env_on(const char *name)
{
	return env_int(name, 1) != 0;
}

static void parse(struct s3h_settings *s)
{
	s->dl_cfg = env_int("SAM3_HIP_DL_CFG", -1);
	s->dlq8_cfg = env_int("SAM3_HIP_DLQ8_CFG", -1);
	s->conv_cfg = env_int("SAM3_HIP_CONV_CFG", -1);
	s->attn_nw = env_int("SAM3_HIP_ATTN_NW", 4);
	s->attn_vdma = env_int("SAM3_HIP_ATTN_VDMA", 1);
	s->sk_mr = s->sk_nt = 0;
	const char *sk = getenv("SAM3_HIP_SK_CFG");
	if (sk && sscanf(sk, "%d,%d", &s->sk_mr, &s->sk_nt) != 2)
		s->sk_mr = s->sk_nt = 0;
	s->q8_expand = env_int("SAM3_HIP_Q8_EXPAND", -1);
	s->q8_f32cast = env_on("SAM3_HIP_Q8_F32CAST");
	s->q8_batch_path = env_int("SAM3_HIP_Q8_BATCH_PATH", 0);
	s->f32_split = env_on("SAM3_HIP_F32_SPLIT");
	s->unpartition_fold = env_on("SAM3_HIP_UNPARTITION_FOLD");
	s->residual_fold = env_on("SAM3_HIP_RESIDUAL_FOLD");
	s->gemm_operand = env_on("SAM3_HIP_GEMM_OPERAND");
	s->qkv_chain = env_on("SAM3_HIP_QKV_CHAIN");
	s->ln_operand = env_on("SAM3_HIP_LN_OPERAND");
	s->permute_operand = env_on("SAM3_HIP_PERMUTE_OPERAND");
	s->partition_fold = env_on("SAM3_HIP_PARTITION_FOLD");
	s->qkv_fold = env_on("SAM3_HIP_QKV_FOLD");
	s->sdpa_merge = env_on("SAM3_HIP_SDPA_MERGE");
	s->ln_gemv_fold = env_on("SAM3_HIP_LN_GEMV_FOLD");
	s->att_gemv_fold = env_on("SAM3_HIP_ATT_GEMV_FOLD");
	s->gemv_tasks = env_on("SAM3_HIP_GEMV_TASKS");
	s->gemv_f32 = env_on("SAM3_HIP_GEMV_F32");
	s->q8_wauto = env_on("SAM3_HIP_Q8_WAUTO");
	const char *rb = getenv("SAM3_HIP_READBACK");
	s->readback_all = rb && rb[0] == 'a' && rb[1] == 'l' && rb[2] == 'l' && !rb[3];
	s->quiet = getenv("SAM3_HIP_QUIET") != NULL;
	s->arena_mb = env_int("SAM3_HIP_ARENA_MB", 0);
}

/* Snapshots are never freed: a reload is rare (tests), and a launch that
 * read the previous pointer may still be using it. */
static _Atomic(const struct s3h_settings *) g_cur;
static pthread_once_t g_once = PTHREAD_ONCE_INIT;

static void first_parse(void)
{
	static struct s3h_settings first;
	parse(&first);
	atomic_store(&g_cur, &first);
}

const struct s3h_settings *s3h_settings(void)
{
	const struct s3h_settings *s = atomic_load_explicit(&g_cur, memory_order_acquire);
	if (s)
		return s;
	pthread_once(&g_once, first_parse);
	return atomic_load(&g_cur);
}

enum sam3_error sam3_hip_reload_settings(void)
{
	pthread_once(&g_once, first_parse);
	struct s3h_settings *s = malloc(sizeof(*s));
	if (!s)
		return SAM3_ENOMEM;
	parse(s);
	atomic_store_explicit(&g_cur, s, memory_order_release);
	return SAM3_OK;
}
