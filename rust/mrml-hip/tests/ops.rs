//! Device tests of the crate, in the form of crates/mrml-tensor/tests/ops_test.rs:
//! each returns at once when no gfx950 device (or no libmrml_hip.so) is there.

use mrml_hip::{HipBuffer, HipDevice};

/// ops_test.rs:165-212: the partitions' candidates hold the exact global
/// top-40 of the penalised logits.
#[test]
fn vocab_topk_contains_exact_global_topk() {
    if !HipDevice::is_available() {
        return;
    }
    const N: usize = 4096;
    const K: usize = 40;
    const PARTITIONS: usize = 8;
    let logits: Vec<f32> = (0..N).map(|i| ((i * 7919 % 65521) as f32) * 0.001 + i as f32 * 1e-7).collect();
    let valid: Vec<u8> = (0..N).map(|i| u8::from(i % 17 != 0)).collect();
    let recent = [31i32, 777, 2049, 4001];
    let mut recent_padded = [0i32; 32];
    recent_padded[..recent.len()].copy_from_slice(&recent);

    let dev = HipDevice::new(0).unwrap();
    let d_logits = HipBuffer::from_host_on(&dev, &logits).unwrap();
    let d_valid = HipBuffer::from_host_on(&dev, &valid).unwrap();
    let d_recent = HipBuffer::from_host_on(&dev, &recent_padded).unwrap();
    let mut d_scores = HipBuffer::<f32>::alloc_on(&dev, PARTITIONS * K).unwrap();
    let mut d_ids = HipBuffer::<i32>::alloc_on(&dev, PARTITIONS * K).unwrap();
    dev.vocab_topk(&d_logits, &d_valid, &d_recent, &mut d_scores, &mut d_ids, N, recent.len(), 10, K, PARTITIONS);
    let mut scores = vec![0.0f32; PARTITIONS * K];
    let mut ids = vec![0i32; PARTITIONS * K];
    d_scores.copy_to_host(&mut scores).unwrap();
    d_ids.copy_to_host(&mut ids).unwrap();

    let mut actual: Vec<_> = scores.into_iter().zip(ids).collect();
    actual.sort_unstable_by(|a, b| b.0.partial_cmp(&a.0).unwrap().then(a.1.cmp(&b.1)));
    actual.truncate(K);
    let mut expected: Vec<_> = logits
        .iter()
        .copied()
        .enumerate()
        .filter(|(id, _)| valid[*id] != 0)
        .map(|(id, mut score)| {
            if recent.contains(&(id as i32)) {
                score -= 1.8;
            }
            (score, id as i32)
        })
        .collect();
    expected.sort_unstable_by(|a, b| b.0.partial_cmp(&a.0).unwrap().then(a.1.cmp(&b.1)));
    expected.truncate(K);
    assert_eq!(actual, expected);
}

/// A Q4_0 product of all-0x88 blocks (every quant 8, i.e. zero) is zero.
#[test]
fn gemv_q4_0_of_zero_blocks_is_zero() {
    if !HipDevice::is_available() {
        return;
    }
    let (rows, cols) = (64usize, 256usize);
    let mut gguf = Vec::with_capacity(rows * cols / 32 * 18);
    for _ in 0..rows * cols / 32 {
        gguf.extend_from_slice(&[0x00, 0x3c]); // f16 1.0
        gguf.extend_from_slice(&[0x88; 16]);
    }
    let dev = HipDevice::new(0).unwrap();
    let w = dev.upload_q4_0(&gguf, rows, cols).unwrap();
    let x = HipBuffer::from_host_on(&dev, &vec![1.0f32; cols]).unwrap();
    let mut y = HipBuffer::<f32>::alloc_on(&dev, rows).unwrap();
    dev.gemv_q4_0(&w, &x, &mut y, rows, cols);
    let mut out = vec![1.0f32; rows];
    y.copy_to_host(&mut out).unwrap();
    assert!(out.iter().all(|v| *v == 0.0));
}
