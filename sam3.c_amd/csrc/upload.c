/*
 * upload.c - bulk host-to-HBM transfers through pinned staging buffers.
 *
 * sam3.c maps its weight file read-only (weight.c:303-474), so the bytes
 * the GPU needs sit in pageable memory the DMA engines cannot read, and
 * registering that mapping as pinned memory is not available. A transfer
 * therefore runs as several lanes. Each lane is a host thread with its
 * own stream and two pinned buffers: while the DMA of one buffer is in
 * flight the thread copies the next chunk of the range into the other.
 * Chunks are dealt to the lanes round-robin, so the host copies run in
 * parallel and consecutive chunks leave on different DMA queues.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "sam3_hip_internal.h"

static int env_int(const char *name, int dflt, int lo, int hi)
{
	const char *s = getenv(name);
	if (!s || !*s)
		return dflt;
	long v = strtol(s, NULL, 10);
	return v < lo ? lo : v > hi ? hi : (int)v;
}

enum sam3_error s3h_stager_init(struct s3h_stager *s, int device)
{
	if (s->lanes)
		return SAM3_OK;
	const int lanes = env_int("SAM3_HIP_UPLOAD_LANES", S3H_STAGE_LANES, 1, S3H_STAGE_MAX_LANES);
	const size_t chunk = (size_t)env_int("SAM3_HIP_UPLOAD_CHUNK_MB", S3H_STAGE_CHUNK_MB, 1, 256)
			     << 20;
	s->device = device;
	s->chunk = chunk;
	enum sam3_error err = SAM3_OK;
	for (int l = 0; l < lanes && err == SAM3_OK; l++) {
		struct s3h_stage_lane *ln = &s->lane[l];
		err = s3h_hip(hipStreamCreateWithFlags((hipStream_t *)&ln->stream, hipStreamNonBlocking),
			      "upload: stream");
		for (int b = 0; b < 2 && err == SAM3_OK; b++) {
			err = s3h_hip(hipHostMalloc((void **)&ln->buf[b], chunk, hipHostMallocDefault),
				      "upload: pinned staging buffer");
			if (err == SAM3_OK)
				err = s3h_hip(hipEventCreateWithFlags((hipEvent_t *)&ln->done[b],
								      hipEventDisableTiming),
					      "upload: event");
		}
		s->lanes = l + 1;
	}
	if (err != SAM3_OK)
		s3h_stager_free(s);
	return err;
}

void s3h_stager_free(struct s3h_stager *s)
{
	for (int l = 0; l < s->lanes; l++) {
		struct s3h_stage_lane *ln = &s->lane[l];
		if (ln->stream)
			(void)hipStreamSynchronize(ln->stream);
		for (int b = 0; b < 2; b++) {
			if (ln->done[b])
				(void)hipEventDestroy(ln->done[b]);
			if (ln->buf[b])
				(void)hipHostFree(ln->buf[b]);
		}
		if (ln->stream)
			(void)hipStreamDestroy(ln->stream);
		memset(ln, 0, sizeof(*ln));
	}
	s->lanes = 0;
}

struct lane_job {
	struct s3h_stager *s;
	int lane;
	int nlanes;
	char *dev;
	const char *host;
	size_t nbytes;
	enum sam3_error err;
};

/* Chunks lane, lane + nlanes, ... of the range; two buffers in turn. */
static void *lane_run(void *arg)
{
	struct lane_job *j = arg;
	struct s3h_stage_lane *ln = &j->s->lane[j->lane];
	const size_t chunk = j->s->chunk;
	enum sam3_error err = s3h_hip(hipSetDevice(j->s->device), "upload: set device");
	int b = 0, used[2] = {0, 0};
	for (size_t c = (size_t)j->lane; err == SAM3_OK && c * chunk < j->nbytes;
	     c += (size_t)j->nlanes) {
		const size_t off = c * chunk;
		const size_t len = j->nbytes - off < chunk ? j->nbytes - off : chunk;
		if (used[b])
			err = s3h_hip(hipEventSynchronize(ln->done[b]), "upload: staging wait");
		if (err != SAM3_OK)
			break;
		memcpy(ln->buf[b], j->host + off, len);
		err = s3h_hip(hipMemcpyAsync(j->dev + off, ln->buf[b], len, hipMemcpyHostToDevice,
					     ln->stream),
			      "upload: copy");
		if (err == SAM3_OK)
			err = s3h_hip(hipEventRecord(ln->done[b], ln->stream), "upload: record");
		used[b] = 1;
		b ^= 1;
	}
	enum sam3_error serr = s3h_hip(hipStreamSynchronize(ln->stream), "upload: sync");
	j->err = err != SAM3_OK ? err : serr;
	return NULL;
}

enum sam3_error s3h_stager_copy(struct s3h_stager *s, void *dev, const void *host, size_t nbytes)
{
	if (!nbytes)
		return SAM3_OK;
	if (!s->lanes) {
		s3h_error("upload: stager not initialised");
		return SAM3_EINVAL;
	}
	const size_t chunks = (nbytes + s->chunk - 1) / s->chunk;
	const int nl = chunks < (size_t)s->lanes ? (int)chunks : s->lanes;
	struct lane_job jobs[S3H_STAGE_MAX_LANES];
	pthread_t th[S3H_STAGE_MAX_LANES];
	int started[S3H_STAGE_MAX_LANES] = {0};
	for (int l = 0; l < nl; l++)
		jobs[l] = (struct lane_job){s, l, nl, (char *)dev, (const char *)host, nbytes,
					    SAM3_OK};
	/* Lane 0 runs on the calling thread; a lane whose thread cannot be
	 * started is run here as well, after lane 0. */
	for (int l = 1; l < nl; l++)
		started[l] = pthread_create(&th[l], NULL, lane_run, &jobs[l]) == 0;
	lane_run(&jobs[0]);
	for (int l = 1; l < nl; l++) {
		if (started[l])
			pthread_join(th[l], NULL);
		else
			lane_run(&jobs[l]);
	}
	for (int l = 0; l < nl; l++)
		if (jobs[l].err != SAM3_OK)
			return jobs[l].err;
	return SAM3_OK;
}
