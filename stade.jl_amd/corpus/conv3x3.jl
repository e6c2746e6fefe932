# conv3x3(loss, xp, w, out, i_nb, i_c, i_k, i_h, i_w)
#
# 3 x 3 convolution (cross-correlation), stride 1, zero padding 1, followed by half
# the squared norm of the output:
#   out[x, y, co, n] = sum_{ci, ky, kx} w[kx, ky, ci, co] * xp[x + kx - 1, y + ky - 1, ci, n]
#   loss += 0.5 * sum(out .^ 2)
# The zero padding is held in the input: xp is the (i_w + 2) x (i_h + 2) image with a
# one-cell zero border, so the tap loop needs no branch.
#
# loss: length-1 output array, accumulated in place
# xp: padded input, (i_w + 2, i_h + 2, i_c, i_nb) column-major
# w: weights, (3, 3, i_c, i_k) column-major
# out: output, (i_w, i_h, i_k, i_nb) column-major, overwritten
# i_nb: batch; i_c: input channels; i_k: output channels; i_h, i_w: image height, width
function conv3x3(loss, xp, w, out, i_nb, i_c, i_k, i_h, i_w)
    i_wp = i_w + 2
    i_hp = i_h + 2
    # one iteration per output pixel (x, y, output channel, sample); the tap sum is carried (rule 1)
    for idx = 1:i_nb * i_k * i_h * i_w
        i_x = mod(idx - 1, i_w) + 1
        i_y = mod(div(idx - 1, i_w), i_h) + 1
        i_co = mod(div(idx - 1, i_w * i_h), i_k) + 1
        i_n = div(idx - 1, i_w * i_h * i_k) + 1
        s = 0.0
        for i_t = 1:i_c * 9
            i_ci = div(i_t - 1, 9) + 1
            i_ky = mod(div(i_t - 1, 3), 3) + 1
            i_kx = mod(i_t - 1, 3) + 1
            s = s + w[((i_co - 1) * i_c + (i_ci - 1)) * 9 + (i_ky - 1) * 3 + i_kx] * xp[(((i_n - 1) * i_c + (i_ci - 1)) * i_hp + (i_y + i_ky - 2)) * i_wp + i_x + i_kx - 1]
        end
        out[idx] = s
    end
    # half the squared norm of the output
    for i_q = 1:i_nb * i_k * i_h * i_w
        loss[1] = loss[1] + 0.5 * out[i_q] ^ 2
    end
    return nothing
end
